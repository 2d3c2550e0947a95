// Head transposes [B, S, H, Dh] <-> [B, H, S, Dh].
//
// Reference: transpose_heads / merge_heads (src/kernels/transpose_heads.rs:49-96)
// copy one Dh-row per 128-thread CTA on a grid [S, H].  Here a row of the
// head layout is just a Dh*elem_bytes run that is contiguous on both sides,
// so the kernel is a permutation of rows done with 16-byte vectors: one
// workgroup streams 4 * 256 vectors of one (b, h) slice, reads and writes
// both fully coalesced within each row.  Element size does not matter (a
// byte-exact copy), so fp32 and bf16 share the kernel.
#include "common.h"

namespace {

template <int VB>
struct VecT;
template <>
struct VecT<16> {
  typedef u32x4 type;
};
template <>
struct VecT<4> {
  typedef uint32_t type;
};

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

// merge == 0: src [B,S,H,row] -> dst [B,H,S,row]   (transpose_heads)
// merge == 1: src [B,H,S,row] -> dst [B,S,H,row]   (merge_heads)
template <int VB>
__device__ void transpose_rows(const char* __restrict__ src, char* __restrict__ dst, int seq,
                               int heads, int row_bytes, int merge) {
  typedef typename VecT<VB>::type V;
  const int vpr = row_bytes / VB;  // vectors per row
  const int bh = blockIdx.y;
  const int b = bh / heads, h = bh - b * heads;
  const long slice = (long)seq * vpr;
  V buf[kUnroll];
  long bhs_off[kUnroll], bsh_off[kUnroll];
  bool ok[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    long flat = ((long)blockIdx.x * kUnroll + u) * kThreads + threadIdx.x;
    ok[u] = flat < slice;
    int s = (int)(flat / vpr);
    int v = (int)(flat - (long)s * vpr);
    bhs_off[u] = ((long)bh * seq + s) * row_bytes + (long)v * VB;
    bsh_off[u] = (((long)b * seq + s) * heads + h) * (long)row_bytes + (long)v * VB;
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u)
    if (ok[u]) buf[u] = *reinterpret_cast<const V*>(src + (merge ? bhs_off[u] : bsh_off[u]));
#pragma unroll
  for (int u = 0; u < kUnroll; ++u)
    if (ok[u]) *reinterpret_cast<V*>(dst + (merge ? bsh_off[u] : bhs_off[u])) = buf[u];
}

}  // namespace

extern "C" __global__ __launch_bounds__(256) void teeny_transpose_heads_v16(
    const char* src, char* dst, int seq, int heads, int row_bytes, int merge) {
  transpose_rows<16>(src, dst, seq, heads, row_bytes, merge);
}

extern "C" __global__ __launch_bounds__(256) void teeny_transpose_heads_v4(
    const char* src, char* dst, int seq, int heads, int row_bytes, int merge) {
  transpose_rows<4>(src, dst, seq, heads, row_bytes, merge);
}

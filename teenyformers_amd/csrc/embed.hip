// Token embedding gather: out[s, :] = weight[ids[s], :].
//
// Reference: token_embed_forward (src/kernels/token_embed.rs:38-76), one CTA
// per token copying BLOCK_D = 1024 columns at a time, ids stored as f32
// (:32, :53).  Here ids may be f32 (the reference's encoding, exact below
// 2^24) or int32, and rows move as 16-byte vectors.  An id outside
// [0, vocab) yields a zero row instead of an out-of-bounds read.
#include "common.h"

namespace {

constexpr int kThreads = 256;

template <int VB, typename ID>
__device__ void embed_rows(const ID* __restrict__ ids, const char* __restrict__ w,
                           char* __restrict__ out, int row_bytes, int vocab) {
  typedef typename std::conditional<VB == 16, u32x4, uint32_t>::type V;
  const int s = blockIdx.y;
  const int off = (blockIdx.x * kThreads + threadIdx.x) * VB;
  if (off >= row_bytes) return;
  long id = (long)ids[s];
  V val;
  if (id >= 0 && id < vocab)
    val = *reinterpret_cast<const V*>(w + id * row_bytes + off);
  else
    val = V{};
  *reinterpret_cast<V*>(out + (long)s * row_bytes + off) = val;
}

}  // namespace

extern "C" __global__ __launch_bounds__(256) void teeny_embed_f32ids_v16(
    const float* ids, const char* w, char* out, int row_bytes, int vocab) {
  embed_rows<16, float>(ids, w, out, row_bytes, vocab);
}
extern "C" __global__ __launch_bounds__(256) void teeny_embed_f32ids_v4(
    const float* ids, const char* w, char* out, int row_bytes, int vocab) {
  embed_rows<4, float>(ids, w, out, row_bytes, vocab);
}
extern "C" __global__ __launch_bounds__(256) void teeny_embed_i32ids_v16(
    const int* ids, const char* w, char* out, int row_bytes, int vocab) {
  embed_rows<16, int>(ids, w, out, row_bytes, vocab);
}
extern "C" __global__ __launch_bounds__(256) void teeny_embed_i32ids_v4(
    const int* ids, const char* w, char* out, int row_bytes, int vocab) {
  embed_rows<4, int>(ids, w, out, row_bytes, vocab);
}

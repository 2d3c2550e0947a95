// Rotary position embedding on x [BH, N_CTX, HEAD_DIM], interleaved pairs.
//
// Reference: rope_forward / rope_backward (src/kernels/rope.rs:57-140), one
// 128-thread CTA per (position, bh) row that recomputes exp, cos and sin for
// every pair of every row.  Here a thread owns one 16-byte vector column
// (position s, pairs v*VN/2 ..) of kHeads consecutive BH rows: it issues the
// kHeads loads first, evaluates its VN/2 (cos, sin) pairs while they are in
// flight, and rotates and stores the kHeads vectors, so the transcendental
// work is amortised over kHeads rows, no LDS table or barrier is needed, and
// the kernel is HBM bound.  (A workgroup-shared LDS table for 16 positions x
// 16 rows ran at 3.8 TB/s at [128, 2048, 64] bf16, this layout at 5.3.)
//
// theta parity with the oracle: inv_freq[k] = fp32(exp_f64(fp32(k) * c)) with
// c = (-2 * ln_base) / HEAD_DIM in fp32 (rope.rs:88), theta = fp32(pos) *
// inv_freq (rope.rs:86-87), cos/sin from the accurate device library.
#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kHeads = 8;  // BH rows per thread

// grid: (ceil(n_ctx / (kThreads / vpr)), ceil(bh / kHeads)); head_dim is a
// power of two (vpr = head_dim / VN vectors per row).
template <typename T>
__device__ void rope_rows(const T* __restrict__ x, T* __restrict__ y, int bh_total, int n_ctx,
                          int head_dim, float ln_base, int backward) {
  constexpr int VN = Vec16<T>::N;  // elements per 16-byte vector (even)
  const int vpr = head_dim / VN;
  const int lg_vpr = __builtin_ctz(vpr);
  const int v = threadIdx.x & (vpr - 1);
  const int s = blockIdx.x * (kThreads >> lg_vpr) + (threadIdx.x >> lg_vpr);
  const int bh0 = blockIdx.y * kHeads;
  if (s >= n_ctx) return;
  const long off0 = ((long)bh0 * n_ctx + s) * head_dim + v * VN;
  const long hstride = (long)n_ctx * head_dim;
  float in[kHeads][VN];
#pragma unroll
  for (int h = 0; h < kHeads; ++h)
    if (bh0 + h < bh_total) Vec16<T>::load(x + off0 + h * hstride, in[h]);

  const float c = rope_c(ln_base, head_dim);
  float cn[VN / 2], sn[VN / 2];
#pragma unroll
  for (int j = 0; j < VN / 2; ++j) {
    rope_cos_sin(s, v * (VN / 2) + j, c, cn[j], sn[j]);
    if (backward) sn[j] = -sn[j];
  }
#pragma unroll
  for (int h = 0; h < kHeads; ++h) {
    if (bh0 + h >= bh_total) continue;
    float out[VN];
#pragma unroll
    for (int j = 0; j < VN / 2; ++j) {
      rope_rotate(in[h][2 * j], in[h][2 * j + 1], cn[j], sn[j], out[2 * j], out[2 * j + 1]);
    }
    Vec16<T>::store(y + off0 + h * hstride, out);
  }
}

}  // namespace

extern "C" __global__ __launch_bounds__(256) void teeny_rope_f32(const float* x, float* y,
                                                                  int bh, int n_ctx, int head_dim,
                                                                  float ln_base, int backward) {
  rope_rows<float>(x, y, bh, n_ctx, head_dim, ln_base, backward);
}

extern "C" __global__ __launch_bounds__(256) void teeny_rope_bf16(const bf16* x, bf16* y, int bh,
                                                                   int n_ctx, int head_dim,
                                                                   float ln_base, int backward) {
  rope_rows<bf16>(x, y, bh, n_ctx, head_dim, ln_base, backward);
}

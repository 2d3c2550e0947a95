// Rotary position embedding on x [BH, N_CTX, HEAD_DIM], interleaved pairs.
//
// Reference: rope_forward / rope_backward (src/kernels/rope.rs:57-140), one
// 128-thread CTA per (position, bh) row that recomputes exp, cos and sin for
// every pair of every row.  Here a workgroup owns kPos positions x kHeads
// rows of BH: it first evaluates the (cos, sin) table for its kPos positions
// into LDS once, then streams kHeads * kPos rows through 16-byte vectors, so
// the transcendental work is amortised over kHeads rows and the kernel is
// HBM bound.
//
// theta parity with the oracle: inv_freq[k] = fp32(exp_f64(fp32(k) * c)) with
// c = (-2 * ln_base) / HEAD_DIM in fp32 (rope.rs:88), theta = fp32(pos) *
// inv_freq (rope.rs:86-87), cos/sin from the accurate device library.
#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kPos = 16;    // positions per workgroup
constexpr int kHeads = 16;  // BH rows per position per workgroup

template <typename T>
__device__ void rope_rows(const T* __restrict__ x, T* __restrict__ y, int bh_total, int n_ctx,
                          int head_dim, float ln_base, int backward) {
  extern __shared__ float2 cs_tab[];  // [kPos][head_dim / 2] (cos, sin)
  const int half = head_dim / 2;
  const int s0 = blockIdx.x * kPos;
  const int bh0 = blockIdx.y * kHeads;
  const float c = (-2.0f * ln_base) / (float)head_dim;
  for (int i = threadIdx.x; i < kPos * half; i += kThreads) {
    int p = i / half, k = i - p * half;
    float inv = (float)exp((double)((float)k * c));
    float theta = (float)(s0 + p) * inv;
    float sn, cn;
    sincosf(theta, &sn, &cn);
    cs_tab[i] = make_float2(cn, sn);
  }
  __syncthreads();

  constexpr int VN = Vec16<T>::N;  // elements per 16-byte vector (even)
  const int vpr = head_dim / VN;   // vectors per row
  const int total = kHeads * kPos * vpr;
  const float sgn = backward ? -1.0f : 1.0f;
  for (int i = threadIdx.x; i < total; i += kThreads) {
    int v = i % vpr;
    int r = i / vpr;
    int p = r % kPos;
    int hh = r / kPos;
    int s = s0 + p, bh = bh0 + hh;
    if (s >= n_ctx || bh >= bh_total) continue;
    long off = ((long)bh * n_ctx + s) * head_dim + v * VN;
    float in[VN], out[VN];
    Vec16<T>::load(x + off, in);
    const float2* cs = cs_tab + p * half + v * (VN / 2);
#pragma unroll
    for (int j = 0; j < VN / 2; ++j) {
      float cn = cs[j].x, sn = sgn * cs[j].y;
      float x0 = in[2 * j], x1 = in[2 * j + 1];
      out[2 * j] = x0 * cn - x1 * sn;
      out[2 * j + 1] = x0 * sn + x1 * cn;
    }
    Vec16<T>::store(y + off, out);
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

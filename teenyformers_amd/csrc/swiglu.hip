// SwiGLU activation on z [M, 2F] (gate || up) -> out [M, F], and its backward.
//
// Reference: swiglu_forward / swiglu_backward (src/kernels/swiglu.rs:56-136),
// one 128-thread CTA per row walking BLOCK_N = 1024 columns.  Here the grid is
// 2-D (column chunks x rows) and every thread moves 16-byte vectors, so the
// kernel is a pure HBM stream (3 x M x F elements forward, 5 x M x F backward).
#include "common.h"

namespace {

constexpr int kThreads = 256;

DEVI float sigmoidf(float g) { return 1.0f / (1.0f + expf(-g)); }

template <typename T, int VEC>
DEVI void ldv(const T* p, float* out) {
  if constexpr (VEC == 1) {
    out[0] = ld(p);
  } else {
    Vec16<T>::load(p, out);
  }
}
template <typename T, int VEC>
DEVI void stv(T* p, const float* in) {
  if constexpr (VEC == 1) {
    st(p, in[0]);
  } else {
    Vec16<T>::store(p, in);
  }
}

template <typename T, int VEC>
__device__ void swiglu_fwd(const T* __restrict__ z, T* __restrict__ out, int M, int F) {
  const int row = blockIdx.y;
  const int col = (blockIdx.x * kThreads + threadIdx.x) * VEC;
  if (row >= M || col >= F) return;
  const T* g = z + (long)row * 2 * F + col;
  float gv[VEC], uv[VEC], o[VEC];
  ldv<T, VEC>(g, gv);
  ldv<T, VEC>(g + F, uv);
#pragma unroll
  for (int j = 0; j < VEC; ++j) o[j] = gv[j] * sigmoidf(gv[j]) * uv[j];
  stv<T, VEC>(out + (long)row * F + col, o);
}

template <typename T, int VEC>
__device__ void swiglu_bwd(const T* __restrict__ grad, const T* __restrict__ z,
                           T* __restrict__ dz, int M, int F) {
  const int row = blockIdx.y;
  const int col = (blockIdx.x * kThreads + threadIdx.x) * VEC;
  if (row >= M || col >= F) return;
  const long zoff = (long)row * 2 * F + col;
  float gv[VEC], uv[VEC], gr[VEC], dg[VEC], du[VEC];
  ldv<T, VEC>(z + zoff, gv);
  ldv<T, VEC>(z + zoff + F, uv);
  ldv<T, VEC>(grad + (long)row * F + col, gr);
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    float sig = sigmoidf(gv[j]);
    float silu = gv[j] * sig;
    float dsilu = sig * (1.0f + gv[j] * (1.0f - sig));
    dg[j] = gr[j] * uv[j] * dsilu;
    du[j] = gr[j] * silu;
  }
  stv<T, VEC>(dz + zoff, dg);
  stv<T, VEC>(dz + zoff + F, du);
}

// Elementwise residual add y = a + b over n values (the reference's sym_add,
// src/layers/mod.rs:36-48, Op::Add): 8 consecutive values per thread as
// 16-byte (bf16) or two 16-byte (fp32) vectors; n % 8 values at the end one
// at a time.
template <typename T>
__device__ void add_kernel(const T* __restrict__ a, const T* __restrict__ b, T* __restrict__ y,
                           long n) {
  const long i = ((long)blockIdx.x * kThreads + threadIdx.x) * 8;
  if (i + 8 <= n) {
    float va[8], vb[8];
    constexpr int N = Vec16<T>::N;
#pragma unroll
    for (int h = 0; h < 8; h += N) {
      Vec16<T>::load(a + i + h, va + h);
      Vec16<T>::load(b + i + h, vb + h);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) va[j] += vb[j];
#pragma unroll
    for (int h = 0; h < 8; h += N) Vec16<T>::store(y + i + h, va + h);
  } else {
    for (long j = i; j < n; ++j) st(y + j, ld(a + j) + ld(b + j));
  }
}

}  // namespace

extern "C" __global__ __launch_bounds__(256) void teeny_add_f32(const float* a, const float* b,
                                                                float* y, long n) {
  add_kernel<float>(a, b, y, n);
}
extern "C" __global__ __launch_bounds__(256) void teeny_add_bf16(const bf16* a, const bf16* b,
                                                                 bf16* y, long n) {
  add_kernel<bf16>(a, b, y, n);
}

#define TEENY_SWIGLU_INST(TN, T, VEC)                                                      \
  extern "C" __global__ __launch_bounds__(256) void teeny_swiglu_fwd_##TN##_v##VEC(       \
      const T* z, T* out, int M, int F) {                                                  \
    swiglu_fwd<T, VEC>(z, out, M, F);                                                      \
  }                                                                                        \
  extern "C" __global__ __launch_bounds__(256) void teeny_swiglu_bwd_##TN##_v##VEC(       \
      const T* grad, const T* z, T* dz, int M, int F) {                                    \
    swiglu_bwd<T, VEC>(grad, z, dz, M, F);                                                 \
  }

TEENY_SWIGLU_INST(f32, float, 4)
TEENY_SWIGLU_INST(f32, float, 1)
TEENY_SWIGLU_INST(bf16, bf16, 8)
TEENY_SWIGLU_INST(bf16, bf16, 1)

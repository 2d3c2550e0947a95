// fp32 linear layer y[M, N] = x[M, K] . w[N, K]^T at the reference's
// precision (teeny-core's Linear behind sym_linear, src/layers/mod.rs:54-58,
// runs in fp32; src/loader.rs:41,66-80 decodes every weight to f32).
//
// teeny_linear_f32 hands its products to hipBLASLt; this kernel is the
// library's own path where hipBLASLt does not take the device, shape or
// stream (a product under graph capture).  Each output is one fp32 fused
// multiply-add chain over k in increasing order, so the result does not
// depend on the tiling.
//
// Tiling: a workgroup of 256 threads owns a 128 x 128 tile of y; 16-deep K
// slices of x and w are staged in LDS transposed (k-major), two buffers, so
// the next slice's global loads are in flight while the current one is
// multiplied; each thread accumulates an 8 x 8 block (rows ty*4 + {0..3} and
// 64 + ty*4 + {0..3}, columns likewise from tx) with 16-byte LDS reads.
// Rows past M or N and k past K load zeros and are never stored.
#include "common.h"

namespace {

constexpr int TM = 128, TN = 128, TK = 16, PAD = 4;

struct Smem {
  float a[2][TK][TM + PAD];  // x slice, k-major
  float b[2][TK][TN + PAD];  // w slice, k-major
};

DEVI f32x4 load4(const float* __restrict__ base, long row, int nrows, int k, int K) {
  if (row < nrows && k < K) return *reinterpret_cast<const f32x4*>(base + row * K + k);
  return f32x4{0.0f, 0.0f, 0.0f, 0.0f};
}

}  // namespace

extern "C" __global__ __launch_bounds__(256) void teeny_gemm_f32_nt(
    const float* __restrict__ x, const float* __restrict__ w, float* __restrict__ y, int M,
    int N, int K) {
  __shared__ Smem sm;
  const int tid = threadIdx.x;
  const int tx = tid & 15, ty = tid >> 4;
  const long m0 = (long)blockIdx.y * TM, n0 = (long)blockIdx.x * TN;

  // staging: each thread brings two 4-float k-runs of x and two of w per
  // slice: tile row r = tid / 4 (+64), k = 4 (tid % 4)
  const int lr = tid >> 2, lk = 4 * (tid & 3);
  auto fetch = [&](int k0, f32x4* ra, f32x4* rb) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      ra[h] = load4(x, m0 + lr + 64 * h, M, k0 + lk, K);
      rb[h] = load4(w, n0 + lr + 64 * h, N, k0 + lk, K);
    }
  };
  auto stash = [&](int buf, const f32x4* ra, const f32x4* rb) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sm.a[buf][lk + j][lr + 64 * h] = ra[h][j];
        sm.b[buf][lk + j][lr + 64 * h] = rb[h][j];
      }
  };

  float acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = 0.0f;

  const int n_slices = (K + TK - 1) / TK;
  f32x4 ra[2], rb[2];
  fetch(0, ra, rb);
  stash(0, ra, rb);
  __syncthreads();
  for (int s = 0; s < n_slices; ++s) {
    const int buf = s & 1;
    if (s + 1 < n_slices) fetch((s + 1) * TK, ra, rb);
#pragma unroll
    for (int k = 0; k < TK; ++k) {
      const f32x4 a0 = *reinterpret_cast<const f32x4*>(&sm.a[buf][k][4 * ty]);
      const f32x4 a1 = *reinterpret_cast<const f32x4*>(&sm.a[buf][k][64 + 4 * ty]);
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(&sm.b[buf][k][4 * tx]);
      const f32x4 b1 = *reinterpret_cast<const f32x4*>(&sm.b[buf][k][64 + 4 * tx]);
      const float av[8] = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
      const float bv[8] = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = __builtin_fmaf(av[i], bv[j], acc[i][j]);
    }
    if (s + 1 < n_slices) stash(buf ^ 1, ra, rb);
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const long m = m0 + (i < 4 ? 4 * ty + i : 64 + 4 * ty + i - 4);
    if (m >= M) continue;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const long n = n0 + 64 * h + 4 * tx;
      float* yr = y + m * N + n;
      if (n + 3 < N && (N & 3) == 0) {
        *reinterpret_cast<f32x4*>(yr) =
            f32x4{acc[i][4 * h], acc[i][4 * h + 1], acc[i][4 * h + 2], acc[i][4 * h + 3]};
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (n + j < N) yr[j] = acc[i][4 * h + j];
      }
    }
  }
}

// RMSNorm and fused residual-add + RMSNorm, forward and backward.
//
// Reference: fused_add_rmsnorm_forward / _backward
// (src/kernels/fused_add_rmsnorm.rs:53-190), one 128-thread CTA per row in two
// passes over HBM with BLOCK_N = 1024.  Here one 64-lane wavefront owns a row
// and keeps it in registers (CH chunks of 64 lanes x VEC elements), so each
// input is read once and each output written once; the sum of squares is a
// wavefront DPP reduction.  The plain RMSNorm of the Llama block
// (src/layers/mod.rs:61-65) is the same kernel without the residual.
//
// Backward: two gradient formulas share the kernel.  REF = true reproduces
// the fused kernel's rstd * w * (dy - h * rstd^2 * dot / N)
// (fused_add_rmsnorm.rs:184), which is the true gradient only when w == 1;
// REF = false is the true RMSNorm gradient rstd * (w * dy - h * rstd^2 *
// dot / N) used for the block's plain norm.
// The reference updates dweight with an unsynchronised
// load + store from every row CTA (fused_add_rmsnorm.rs:182, :187), a race
// when M > 1.  Here each workgroup writes per-column partial sums of
// dy * h * rstd to a workspace and a second kernel adds the column sums to
// dweight in a fixed order (deterministic).
#include "common.h"

namespace {

constexpr int kWaves = 4;

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

// y = h * rstd * w with h = x (+ res); h stored if h_out != nullptr.
// Rows are strided over the grid's wavefronts (the host launches at most
// 1024 workgroups), and while a wavefront reduces and stores one
// row, its next row's loads are in flight (when two rows fit in registers),
// so reads and writes stream together as in a copy: 8192 rows of 2048 bf16
// took 13.4 us with one row per wavefront and every row's loads first, 11.2
// us this way (a device copy of the same bytes: 10.7 us); rows of 4096,
// 23.6 and 20.7 us (copy 20.0).  The arithmetic per row is unchanged.
// RES: the fused form (h = x + res, stored to h_out); a separate instance
// from the plain norm, so neither carries the other's registers.  FULL: N is
// exactly CH x 64 lanes x VEC, so no chunk needs a bounds test and a row's
// loads are issued back to back (with the tests the compiler branches around
// each chunk's loads: 13.0 against 11.2 us at 8192 x 2048 bf16).
template <typename T, int VEC, int CH, bool RES, bool FULL>
__device__ __forceinline__ void rmsnorm_fwd_row(const T* __restrict__ x, const T* __restrict__ res,
                                                T* __restrict__ y, T* __restrict__ h_out,
                                                float* __restrict__ rstd, const T* __restrict__ w,
                                                int M, int N, float eps) {
  constexpr bool kPipe = CH * VEC <= 64;  // two rows in registers
  const int lane = threadIdx.x & 63;
  const int stride = gridDim.x * kWaves;
  int row = blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= M) return;
  // up to 4 chunks the weights are read once, before the rows (wider rows
  // would double the registers of a wavefront)
  constexpr bool kPre = CH <= 4;
  float wv[kPre ? CH : 1][VEC];
  if constexpr (kPre) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      int idx = (c * 64 + lane) * VEC;
      if (FULL || idx < N) ldv<T, VEC>(w + idx, wv[c]);
    }
  }
  // h = x (+ res) of one row, in fp32
  auto load_row = [&](int r, float (*hv)[VEC]) __attribute__((always_inline)) {
    const long base = (long)r * N;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      int idx = (c * 64 + lane) * VEC;
      if (FULL || idx < N) {
        ldv<T, VEC>(x + base + idx, hv[c]);
        if constexpr (RES) {
          float rv[VEC];
          ldv<T, VEC>(res + base + idx, rv);
#pragma unroll
          for (int j = 0; j < VEC; ++j) hv[c][j] += rv[j];
        }
      }
    }
  };
  float hv[CH][VEC];
  float nx[kPipe ? CH : 1][VEC];
  load_row(row, hv);
  for (;;) {
    const int next = row + stride;
    if constexpr (kPipe) {
      if (next < M) load_row(next, nx);
    }
    const long base = (long)row * N;
    float sq = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      int idx = (c * 64 + lane) * VEC;
      if (FULL || idx < N) {
#pragma unroll
        for (int j = 0; j < VEC; ++j) sq += hv[c][j] * hv[c][j];
        if constexpr (RES) {
          stv<T, VEC>(h_out + base + idx, hv[c]);
          // The second pass of the reference reloads h from its storage type.
#pragma unroll
          for (int j = 0; j < VEC; ++j) hv[c][j] = (float)(T)hv[c][j];
        }
      }
    }
    sq = wave_sum(sq);
    const float rs = 1.0f / sqrtf(sq * (1.0f / (float)N) + eps);
    if (lane == 0 && rstd) rstd[row] = rs;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      int idx = (c * 64 + lane) * VEC;
      if (FULL || idx < N) {
        float out[VEC];
        float wl[VEC];
        if constexpr (kPre) {
#pragma unroll
          for (int j = 0; j < VEC; ++j) wl[j] = wv[c][j];
        } else {
          ldv<T, VEC>(w + idx, wl);
        }
#pragma unroll
        for (int j = 0; j < VEC; ++j) out[j] = hv[c][j] * rs * wl[j];
        stv<T, VEC>(y + base + idx, out);
      }
    }
    if (next >= M) break;
    row = next;
    if constexpr (kPipe) {
#pragma unroll
      for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int j = 0; j < VEC; ++j) hv[c][j] = nx[c][j];
    } else {
      load_row(row, hv);
    }
  }
}

// Rows are strided over a fixed number of workgroups; each wave keeps its
// dweight partial in registers and the 4 waves combine through LDS.
template <typename T, int VEC, int CH, bool REF>
__device__ void rmsnorm_bwd_rows(const T* __restrict__ dy, const T* __restrict__ h,
                                 T* __restrict__ dx, T* __restrict__ dres,
                                 float* __restrict__ dw_part, const T* __restrict__ w,
                                 const float* __restrict__ rstd, int M, int N) {
  __shared__ float red[kWaves - 1][CH * 64 * VEC];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  float dwacc[CH][VEC];
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int j = 0; j < VEC; ++j) dwacc[c][j] = 0.0f;
  const float n_inv = 1.0f / (float)N;
  for (int row = blockIdx.x * kWaves + wave; row < M; row += gridDim.x * kWaves) {
    const long base = (long)row * N;
    const float rs = rstd[row];
    float dyv[CH][VEC], hv[CH][VEC], wv[CH][VEC];
    float dot = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      int idx = (c * 64 + lane) * VEC;
      if (idx < N) {
        ldv<T, VEC>(dy + base + idx, dyv[c]);
        ldv<T, VEC>(h + base + idx, hv[c]);
        ldv<T, VEC>(w + idx, wv[c]);
#pragma unroll
        for (int j = 0; j < VEC; ++j) dot += dyv[c][j] * wv[c][j] * hv[c][j];
      }
    }
    dot = wave_sum(dot);
    const float rs2 = rs * rs;
    const float sc = dot * n_inv;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      int idx = (c * 64 + lane) * VEC;
      if (idx < N) {
        float g[VEC];
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          g[j] = REF ? rs * wv[c][j] * (dyv[c][j] - hv[c][j] * rs2 * sc)
                     : rs * (wv[c][j] * dyv[c][j] - hv[c][j] * rs2 * sc);
          dwacc[c][j] += dyv[c][j] * hv[c][j] * rs;
        }
        stv<T, VEC>(dx + base + idx, g);
        if (dres) stv<T, VEC>(dres + base + idx, g);
      }
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int c = 0; c < CH; ++c)
#pragma unroll
      for (int j = 0; j < VEC; ++j) red[wave - 1][(c * 64 + lane) * VEC + j] = dwacc[c][j];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      int idx = (c * 64 + lane) * VEC;
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        float s = dwacc[c][j];
#pragma unroll
        for (int wv2 = 0; wv2 < kWaves - 1; ++wv2) s += red[wv2][idx + j];
        if (idx + j < N) dw_part[(long)blockIdx.x * N + idx + j] = s;
      }
    }
  }
}

}  // namespace

// dweight[n] += sum over workgroups of the partials (fixed order).
extern "C" __global__ __launch_bounds__(256) void teeny_rmsnorm_dw_reduce_f32(
    const float* part, float* dw, int nparts, int N) {
  int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  float s = 0.0f;
  for (int p = 0; p < nparts; ++p) s += part[(long)p * N + n];
  dw[n] = dw[n] + s;
}

extern "C" __global__ __launch_bounds__(256) void teeny_rmsnorm_dw_reduce_bf16(
    const float* part, bf16* dw, int nparts, int N) {
  int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  float s = 0.0f;
  for (int p = 0; p < nparts; ++p) s += part[(long)p * N + n];
  dw[n] = (bf16)((float)dw[n] + s);
}

// Few rows (a decode step's M = batch): one 256-thread workgroup per row, so
// a row's loads are spread over four wavefronts instead of serialised in one;
// the four wavefront sums are added in a fixed order.  PARTS: x is the sum of
// n_parts fp32 slabs [n_parts][M][N] (a linear layer split over K), rounded
// to T as the unsplit product would be stored.
template <typename T, int VEC, int CH, bool PARTS = false, int NT = 256>
__device__ void rmsnorm_fwd_row_wg(const T* __restrict__ x, const T* __restrict__ res,
                                   T* __restrict__ y, T* __restrict__ h_out,
                                   float* __restrict__ rstd, const T* __restrict__ w, int N,
                                   float eps, const float* __restrict__ xparts = nullptr,
                                   int n_parts = 0) {
  __shared__ float part[NT / 64];
  const int tid = threadIdx.x;
  const int row = blockIdx.x;
  const long base = (long)row * N;
  // the weight and residual loads go out first, then x (or its slabs): the
  // row waits for memory once
  float wv[CH][VEC], rv[CH][VEC];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    int idx = (c * NT + tid) * VEC;
    if (idx < N) {
      ldv<T, VEC>(w + idx, wv[c]);
      if (res) ldv<T, VEC>(res + base + idx, rv[c]);
    }
  }
  float hv[CH][VEC];
  float sq = 0.0f;
  if constexpr (PARTS) {  // every chunk's slab loads in flight together
    int off[CH];            // chunks past the row re-read its first element
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int idx = (c * NT + tid) * VEC;
      off[c] = idx < N ? idx : 0;
    }
    ld_parts<T, VEC, CH>(xparts + base, (long)gridDim.x * N, n_parts, hv, off);
  }
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    int idx = (c * NT + tid) * VEC;
    if (idx < N) {
      if constexpr (!PARTS) ldv<T, VEC>(x + base + idx, hv[c]);
      if (res) {
#pragma unroll
        for (int j = 0; j < VEC; ++j) hv[c][j] += rv[c][j];
      }
#pragma unroll
      for (int j = 0; j < VEC; ++j) sq += hv[c][j] * hv[c][j];
      if (h_out) {
        stv<T, VEC>(h_out + base + idx, hv[c]);
#pragma unroll
        for (int j = 0; j < VEC; ++j) hv[c][j] = (float)(T)hv[c][j];
      }
    }
  }
  sq = wave_sum(sq);
  if ((tid & 63) == 0) part[tid >> 6] = sq;
  __syncthreads();
  if constexpr (NT == 256) {
    sq = (part[0] + part[1]) + (part[2] + part[3]);
  } else {
    static_assert(NT == 512, "256 or 512 threads");
    sq = ((part[0] + part[1]) + (part[2] + part[3])) + ((part[4] + part[5]) + (part[6] + part[7]));
  }
  const float rs = 1.0f / sqrtf(sq * (1.0f / (float)N) + eps);
  if (tid == 0 && rstd) rstd[row] = rs;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    int idx = (c * NT + tid) * VEC;
    if (idx < N) {
      float out[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) out[j] = hv[c][j] * rs * wv[c][j];
      stv<T, VEC>(y + base + idx, out);
    }
  }
}

#define TEENY_NORM_WG_INST(TN, T, VEC, CH)                                                      \
  extern "C" __global__ __launch_bounds__(256) void teeny_rmsnorm_fwd_wg_##TN##_v##VEC##_c##CH( \
      const T* x, const T* res, T* y, T* h, float* rstd, const T* w, int M, int N, float eps) { \
    rmsnorm_fwd_row_wg<T, VEC, CH>(x, res, y, h, rstd, w, N, eps);                              \
  }
#define TEENY_NORM_PARTS_INST(TN, T, VEC, CH)                                                 \
  extern "C" __global__ __launch_bounds__(256) void                                            \
      teeny_addnorm_parts_fwd_##TN##_v##VEC##_c##CH(const float* parts, int n_parts,           \
                                                    const T* res, T* y, T* h, float* rstd,     \
                                                    const T* w, int M, int N, float eps) {     \
    rmsnorm_fwd_row_wg<T, VEC, CH, true>(nullptr, res, y, h, rstd, w, N, eps, parts, n_parts); \
  }
TEENY_NORM_PARTS_INST(f32, float, 4, 1)
TEENY_NORM_PARTS_INST(f32, float, 4, 2)
TEENY_NORM_PARTS_INST(f32, float, 4, 4)
TEENY_NORM_PARTS_INST(bf16, bf16, 8, 1)
TEENY_NORM_PARTS_INST(bf16, bf16, 8, 2)
TEENY_NORM_PARTS_INST(bf16, bf16, 8, 4)
TEENY_NORM_WG_INST(f32, float, 4, 1)
TEENY_NORM_WG_INST(f32, float, 4, 2)
TEENY_NORM_WG_INST(f32, float, 4, 4)
TEENY_NORM_WG_INST(bf16, bf16, 8, 1)
TEENY_NORM_WG_INST(bf16, bf16, 8, 2)
TEENY_NORM_WG_INST(bf16, bf16, 8, 4)

// 512 threads per row: bf16 rows of 4096 (one 8-element vector per thread,
// twice the loads in flight of the 256-thread kernels)
extern "C" __global__ __launch_bounds__(512) void teeny_rmsnorm_fwd_wg_bf16_v8_c1_t512(
    const bf16* x, const bf16* res, bf16* y, bf16* h, float* rstd, const bf16* w, int M, int N,
    float eps) {
  rmsnorm_fwd_row_wg<bf16, 8, 1, false, 512>(x, res, y, h, rstd, w, N, eps);
}
extern "C" __global__ __launch_bounds__(512) void teeny_addnorm_parts_fwd_bf16_v8_c1_t512(
    const float* parts, int n_parts, const bf16* res, bf16* y, bf16* h, float* rstd, const bf16* w,
    int M, int N, float eps) {
  rmsnorm_fwd_row_wg<bf16, 8, 1, true, 512>(nullptr, res, y, h, rstd, w, N, eps, parts, n_parts);
}

#define TEENY_NORM_FWD_INST(TN, T, VEC, CH, FULL, SFX)                                           \
  extern "C" __global__ __launch_bounds__(256) void                                              \
      teeny_rmsnorm_fwd_##TN##_v##VEC##_c##CH##SFX(const T* x, const T* res, T* y, T* h,         \
                                                   float* rstd, const T* w, int M, int N,        \
                                                   float eps) {                                  \
    rmsnorm_fwd_row<T, VEC, CH, false, FULL>(x, res, y, h, rstd, w, M, N, eps);                  \
  }                                                                                              \
  extern "C" __global__ __launch_bounds__(256) void                                              \
      teeny_addnorm_fwd_##TN##_v##VEC##_c##CH##SFX(const T* x, const T* res, T* y, T* h,         \
                                                   float* rstd, const T* w, int M, int N,        \
                                                   float eps) {                                  \
    rmsnorm_fwd_row<T, VEC, CH, true, FULL>(x, res, y, h, rstd, w, M, N, eps);                   \
  }
#define TEENY_NORM_INST(TN, T, VEC, CH)                                                          \
  TEENY_NORM_FWD_INST(TN, T, VEC, CH, false, )                                                   \
  TEENY_NORM_FWD_INST(TN, T, VEC, CH, true, _full)                                               \
  extern "C" __global__ __launch_bounds__(256) void teeny_rmsnorm_bwd_##TN##_v##VEC##_c##CH(    \
      const T* dy, const T* h, T* dx, T* dres, float* dw_part, const T* w, const float* rstd,    \
      int M, int N) {                                                                            \
    rmsnorm_bwd_rows<T, VEC, CH, false>(dy, h, dx, dres, dw_part, w, rstd, M, N);                \
  }                                                                                              \
  extern "C" __global__ __launch_bounds__(256) void teeny_addnorm_bwd_##TN##_v##VEC##_c##CH(    \
      const T* dy, const T* h, T* dx, T* dres, float* dw_part, const T* w, const float* rstd,    \
      int M, int N) {                                                                            \
    rmsnorm_bwd_rows<T, VEC, CH, true>(dy, h, dx, dres, dw_part, w, rstd, M, N);                 \
  }

#define TEENY_NORM_ALL_CH(TN, T, VEC) \
  TEENY_NORM_INST(TN, T, VEC, 1)      \
  TEENY_NORM_INST(TN, T, VEC, 2)      \
  TEENY_NORM_INST(TN, T, VEC, 4)      \
  TEENY_NORM_INST(TN, T, VEC, 8)      \
  TEENY_NORM_INST(TN, T, VEC, 16)

TEENY_NORM_ALL_CH(f32, float, 4)
TEENY_NORM_ALL_CH(f32, float, 1)
TEENY_NORM_ALL_CH(bf16, bf16, 8)
TEENY_NORM_ALL_CH(bf16, bf16, 1)

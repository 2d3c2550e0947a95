// Skinny linear layers of a decode step: y[M, N] = x[M, K] . W[N, K]^T with
// M <= 16 (one new token per sequence), bf16 in, fp32 accumulation.
//
// Reference: sym_linear (src/layers/mod.rs:54-58) lowers to the external
// teeny-core Linear, y = x W^T with W in HF [out, in] layout
// (src/loader.rs:19-27).  With M <= 16 the product is bound by streaming W
// from HBM once.
//
// A workgroup of 8 wavefronts owns 128 output features (16 W rows per
// wavefront) and one K range.  x is staged in LDS in 512-wide K chunks,
// double-buffered and shared by the eight wavefronts, so the L2 -> CU traffic
// for x is an eighth of W's (reading x from L2 once per 16 rows capped the W
// stream near 4 TB/s).  A wavefront loads the four 128-wide K steps of a
// chunk for its 16 rows into registers (lane (r = lane % 16, g = lane / 16):
// 64 contiguous bytes of row r at k = 128 j + 32 g), then issues
// v_mfma_f32_16x16x32_bf16 with W as A and x^T, read from LDS at the same k,
// as B.  Rows past M repeat row M - 1 and their outputs are dropped.
//
// Outputs:
//   teeny_linear_sk_bf16        one K range (K), y bf16 [M, N]
//   teeny_linear_sk_swiglu_bf16 wavefronts 0-3 compute gate rows, 4-7 the
//                               matching up rows of the fused gate_up weight;
//                               y [M, F] = silu(gate) * up, both rounded to
//                               bf16 first as the unfused path stores them
//                               (src/layers/ffn.rs:47-56, swiglu.rs:68-85)
//   teeny_linear_sk_part_bf16   blockIdx.y = K split; fp32 partial sums
//                               part[split][M][N], added in split order by
//                               the consumer (the residual-add norm or the
//                               QKV split), which rounds the sum to bf16 as
//                               the unsplit product would be stored.
#include "cdna4.h"

namespace {

constexpr int NW = 8;            // wavefronts per workgroup
constexpr int XC = 512;          // K per staged x chunk (4 steps of 128)
constexpr int XS = XC * 2 + 16;  // bytes per LDS x row; the pad spreads rows over banks

DEVI f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

enum SkMode { SK_BF16, SK_SWIGLU, SK_PART };

// K % 128 == 0; the K range of a workgroup is [blockIdx.y * KC, +KC) with
// KC % 128 == 0 (or KC == K); its last chunk may hold fewer than 4 steps.
template <SkMode MODE>
__device__ void linear_sk(const bf16* __restrict__ x, const bf16* __restrict__ w,
                          void* __restrict__ out, int M, int N, int K, int KC) {
  __shared__ __attribute__((aligned(16))) char xs[2][16 * XS];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  // first W row of this wavefront
  int row0;
  if constexpr (MODE == SK_SWIGLU)
    row0 = blockIdx.x * (8 * NW) + 16 * (wave % (NW / 2)) + (wave / (NW / 2)) * N;  // N = F
  else
    row0 = blockIdx.x * (16 * NW) + 16 * wave;
  const int kb = blockIdx.y * KC, ke = min(kb + KC, K);
  const int nch = (ke - kb + XC - 1) / XC;
  const bf16* wr = w + (long)(row0 + r) * K + 32 * g;

  // x staging: a chunk row is 64 16-byte pieces (16 per 128-wide step);
  // thread t copies pieces P = t % TP + TP j of row t / TP
  constexpr int TP = NW * 64 / 16, XJ = 64 / TP;
  const int xm = tid / TP, xp = tid % TP;
  const bf16* xsrc = x + (long)min(xm, M - 1) * K + 8 * xp;
  u32x4 xv[XJ];
  auto xload = [&](int k0, int nsteps) {
#pragma unroll
    for (int j = 0; j < XJ; ++j)
      if ((xp + TP * j) / 16 < nsteps)
        xv[j] = *reinterpret_cast<const u32x4*>(xsrc + k0 + 8 * TP * j);
  };
  auto xstore = [&](int buf, int nsteps) {
#pragma unroll
    for (int j = 0; j < XJ; ++j)
      if ((xp + TP * j) / 16 < nsteps)
        *reinterpret_cast<u32x4*>(xs[buf] + xm * XS + 16 * (xp + TP * j)) = xv[j];
  };
  auto steps_of = [&](int k0) { return min(4, (ke - k0) >> 7); };

  xload(kb, steps_of(kb));
  xstore(0, steps_of(kb));
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int c = 0; c < nch; ++c) {
    const int k0 = kb + c * XC;
    const int ns = steps_of(k0);
    u32x4 a[4][4];
    if (ns == 4) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          a[j][q] = *reinterpret_cast<const u32x4*>(wr + k0 + 128 * j + 8 * q);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (j < ns)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            a[j][q] = *reinterpret_cast<const u32x4*>(wr + k0 + 128 * j + 8 * q);
    }
    if (c + 1 < nch) xload(k0 + XC, steps_of(k0 + XC));
    // chunk c is in xs[c & 1]; every wavefront is done with chunk c - 1
    __syncthreads();
    const char* xb = xs[c & 1] + r * XS + 64 * g;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (j < ns)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          acc = mfma16(a[j][q], *reinterpret_cast<const u32x4*>(xb + 256 * j + 16 * q), acc);
    if (c + 1 < nch) xstore((c + 1) & 1, steps_of(k0 + XC));
  }

  // lane: token r, features f0 + 4 g + i of the wavefront's 16
  if constexpr (MODE == SK_SWIGLU) {
    __syncthreads();  // done with xs: reuse it for the up halves
    f32x4* up = reinterpret_cast<f32x4*>(xs[0]);
    if (wave >= NW / 2) up[(wave - NW / 2) * 64 + lane] = acc;
    __syncthreads();
    if (wave < NW / 2 && r < M) {
      const f32x4 u = up[wave * 64 + lane];
      float o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float gate = (float)(bf16)acc[i], upv = (float)(bf16)u[i];
        o[i] = gate * (1.0f / (1.0f + expf(-gate))) * upv;
      }
      bf16* y = (bf16*)out + (long)r * N + blockIdx.x * (8 * NW) + 16 * wave + 4 * g;
      *reinterpret_cast<u32x2*>(y) = u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
    }
  } else if (r < M) {
    if constexpr (MODE == SK_BF16) {
      bf16* y = (bf16*)out + (long)r * N + row0 + 4 * g;
      *reinterpret_cast<u32x2*>(y) =
          u32x2{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])};
    } else {
      float* p = (float*)out + ((long)blockIdx.y * M + r) * N + row0 + 4 * g;
      *reinterpret_cast<f32x4*>(p) = acc;
    }
  }
}

}  // namespace

extern "C" __global__ __launch_bounds__(NW * 64) void teeny_linear_sk_bf16(
    const bf16* x, const bf16* w, bf16* y, int M, int N, int K) {
  linear_sk<SK_BF16>(x, w, y, M, N, K, K);
}

extern "C" __global__ __launch_bounds__(NW * 64) void teeny_linear_sk_swiglu_bf16(
    const bf16* x, const bf16* w, bf16* y, int M, int F, int K) {
  linear_sk<SK_SWIGLU>(x, w, y, M, F, K, K);
}

extern "C" __global__ __launch_bounds__(NW * 64) void teeny_linear_sk_part_bf16(
    const bf16* x, const bf16* w, float* part, int M, int N, int K, int KC) {
  linear_sk<SK_PART>(x, w, part, M, N, K, KC);
}

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
//   teeny_linear_sl_*           the same three, same products and bits, for
//                               a weight rewritten once into the streaming
//                               layout by teeny_linear_stream_layout_bf16:
//                               each W load instruction of a wavefront reads
//                               1 KiB contiguous instead of 64 pieces of 16
//                               bytes over 16 rows (measured 3-9 % faster on
//                               the large decode weights, which stream from
//                               HBM).
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
// Load (j, q) of lane (r, g) holds k = 128 j + 32 g + 8 q .. + 7 of W row
// row0 + r, and the product (j, q) reads x at the same k.  SL: w is in the
// streaming layout (teeny_linear_stream_layout_bf16), [N/16][K/128][q 4]
// [g 4][r 16][8] holding exactly those pieces in lane order, so a load
// instruction reads one contiguous KiB (row-major: 64 pieces of 16 bytes
// over 16 rows) and a chunk of 16 rows is 16 KiB; the products and their
// order are the same, so are the results.
// PF: the next chunk's W is loaded into a second register set before this
// chunk's products, and the x barrier leaves those loads in flight.
template <SkMode MODE, bool SL, bool PF>
__device__ __forceinline__ void linear_sk(const bf16* __restrict__ x, const bf16* __restrict__ w,
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
  // element offset of W load (j, q) at chunk start k0: wr + k0 * KM + woff(j, q)
  const bf16* wr = SL ? w + (long)(row0 / 16) * (K / 128) * 2048 + lane * 8
                      : w + (long)(row0 + r) * K + 32 * g;
  constexpr int KM = SL ? 16 : 1;
  auto woff = [](int j, int q) { return SL ? 2048 * j + 512 * q : 128 * j + 8 * q; };
  // LDS byte offset of this lane's x piece for product (j, q): the same k
  const int xoff = 64 * g;
  auto xro = [](int j, int q) { return 256 * j + 16 * q; };

  // x staging: a chunk row is 64 16-byte pieces (16 per 128-wide step);
  // thread t copies pieces P = t % TP + TP j of row t / TP
  constexpr int TP = NW * 64 / 16, XJ = 64 / TP;
  const int xm = tid / TP, xp = tid % TP;
  const bf16* xsrc = x + (long)min(xm, M - 1) * K + 8 * xp;
  u32x4 xv[XJ];
  auto xload = [&](int k0, int nsteps) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < XJ; ++j)
      if ((xp + TP * j) / 16 < nsteps)
        xv[j] = *reinterpret_cast<const u32x4*>(xsrc + k0 + 8 * TP * j);
  };
  auto xstore = [&](int buf, int nsteps) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < XJ; ++j)
      if ((xp + TP * j) / 16 < nsteps)
        *reinterpret_cast<u32x4*>(xs[buf] + xm * XS + 16 * (xp + TP * j)) = xv[j];
  };
  auto steps_of = [&](int k0) { return min(4, (ke - k0) >> 7); };
  // chunk c is in xs[c & 1]; every wavefront is done with chunk c - 1.  With
  // PF only the LDS stores are waited for: __syncthreads would also wait for
  // the next chunk's W loads in flight (vmcnt(0)).
  auto sync = [&]() __attribute__((always_inline)) {
    if constexpr (PF) {
      __builtin_amdgcn_s_waitcnt(kVmWaitLgkm0<63>());
      barrier_only();
    } else {
      __syncthreads();
    }
  };

  // (macros, not lambdas over the register arrays: passed by reference, the
  // arrays were kept in scratch memory)
#define TEENY_SK_WLOAD(A, K0, NS)                                                              \
  do {                                                                                         \
    if ((NS) == 4) {                                                                           \
      _Pragma("unroll") for (int j = 0; j < 4; ++j)                                            \
        _Pragma("unroll") for (int q = 0; q < 4; ++q)                                          \
          A[j][q] = *reinterpret_cast<const u32x4*>(wr + (long)(K0) * KM + woff(j, q));        \
    } else {                                                                                   \
      _Pragma("unroll") for (int j = 0; j < 4; ++j) if (j < (NS))                              \
        _Pragma("unroll") for (int q = 0; q < 4; ++q)                                          \
          A[j][q] = *reinterpret_cast<const u32x4*>(wr + (long)(K0) * KM + woff(j, q));        \
    }                                                                                          \
  } while (0)
#define TEENY_SK_CHUNK(C, A, AN)                                                               \
  do {                                                                                         \
    const int k0 = kb + (C) * XC;                                                              \
    const int ns = steps_of(k0);                                                               \
    if constexpr (PF) {                                                                        \
      /* x first: the x store below waits for the x loads only */                             \
      if ((C) + 1 < nch) {                                                                     \
        xload(k0 + XC, steps_of(k0 + XC));                                                     \
        TEENY_SK_WLOAD(AN, k0 + XC, steps_of(k0 + XC));                                        \
      }                                                                                        \
    } else {                                                                                   \
      TEENY_SK_WLOAD(A, k0, ns);                                                               \
      if ((C) + 1 < nch) xload(k0 + XC, steps_of(k0 + XC));                                    \
    }                                                                                          \
    sync();                                                                                    \
    const char* xb = xs[(C) & 1] + r * XS + xoff;                                              \
    _Pragma("unroll") for (int j = 0; j < 4; ++j) if (j < ns)                                  \
      _Pragma("unroll") for (int q = 0; q < 4; ++q)                                            \
        acc = mfma16(A[j][q], *reinterpret_cast<const u32x4*>(xb + xro(j, q)), acc);           \
    if ((C) + 1 < nch) xstore(((C) + 1) & 1, steps_of(k0 + XC));                               \
  } while (0)

  xload(kb, steps_of(kb));
  xstore(0, steps_of(kb));
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  u32x4 a0[4][4], a1[4][4];
  if constexpr (PF) {
    TEENY_SK_WLOAD(a0, kb, steps_of(kb));
    int c = 0;
    for (; c + 1 < nch; c += 2) {
      TEENY_SK_CHUNK(c, a0, a1);
      TEENY_SK_CHUNK(c + 1, a1, a0);
    }
    if (c < nch) TEENY_SK_CHUNK(c, a0, a1);
  } else {
    for (int c = 0; c < nch; ++c) TEENY_SK_CHUNK(c, a0, a1);
  }
#undef TEENY_SK_CHUNK
#undef TEENY_SK_WLOAD

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
  linear_sk<SK_BF16, false, false>(x, w, y, M, N, K, K);
}

extern "C" __global__ __launch_bounds__(NW * 64) void teeny_linear_sk_swiglu_bf16(
    const bf16* x, const bf16* w, bf16* y, int M, int F, int K) {
  linear_sk<SK_SWIGLU, false, false>(x, w, y, M, F, K, K);
}

extern "C" __global__ __launch_bounds__(NW * 64) void teeny_linear_sk_part_bf16(
    const bf16* x, const bf16* w, float* part, int M, int N, int K, int KC) {
  linear_sk<SK_PART, false, false>(x, w, part, M, N, K, KC);
}

// Streaming-layout weights.  The next chunk's W loads are issued ahead where
// that measured faster at the Llama-3-8B decode shapes (the fused gate_up +
// SwiGLU 9 %, the 128256-row lm_head 3 %); the K-split form keeps one chunk
// in flight (with the look-ahead it ran 0-5 % slower).
extern "C" __global__ __launch_bounds__(NW * 64) void teeny_linear_sl_bf16(
    const bf16* x, const bf16* w, bf16* y, int M, int N, int K) {
  linear_sk<SK_BF16, true, true>(x, w, y, M, N, K, K);
}

extern "C" __global__ __launch_bounds__(NW * 64) void teeny_linear_sl_swiglu_bf16(
    const bf16* x, const bf16* w, bf16* y, int M, int F, int K) {
  linear_sk<SK_SWIGLU, true, true>(x, w, y, M, F, K, K);
}

extern "C" __global__ __launch_bounds__(NW * 64) void teeny_linear_sl_part_bf16(
    const bf16* x, const bf16* w, float* part, int M, int N, int K, int KC) {
  linear_sk<SK_PART, true, false>(x, w, part, M, N, K, KC);
}

// Row-major W [N, K] -> the streaming layout [N/16][K/128][q][g][r][8]:
// piece p = (((nb * K/128 + ks) * 4 + q) * 4 + g) * 16 + r holds
// W[16 nb + r][128 ks + 32 g + 8 q .. + 7]; thread t moves piece t
// (N % 16 == 0, K % 128 == 0, N * K / 8 pieces).
extern "C" __global__ __launch_bounds__(256) void teeny_linear_stream_layout_bf16(
    const bf16* __restrict__ w, bf16* __restrict__ wl, int N, int K, long n_pieces) {
  const long p = (long)blockIdx.x * 256 + threadIdx.x;
  if (p >= n_pieces) return;
  const int r = (int)(p & 15), g = (int)((p >> 4) & 3), q = (int)((p >> 6) & 3);
  const long blk = p >> 8;
  const int KS = K / 128;
  const long nb = blk / KS;
  const int ks = (int)(blk - nb * KS);
  const long row = nb * 16 + r;
  const int k = 128 * ks + 32 * g + 8 * q;
  *reinterpret_cast<u32x4*>(wl + p * 8) = *reinterpret_cast<const u32x4*>(w + row * K + k);
}

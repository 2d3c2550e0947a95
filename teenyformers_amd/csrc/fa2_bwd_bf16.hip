// bf16 flash-attention 2 backward on CDNA4 matrix cores (gfx950).
//
// Reference semantics: flash_attn2_causal_bwd (src/kernels/flash_attn2.rs:135-203)
// and flash_attn2_backward (:209-279):
//   P = exp(scale * Q K^T - LSE), dV = P^T dO, dP = dO V^T,
//   dS = P o (dP - Delta) with Delta = rowsum(O o dO), dQ = scale dS K,
//   dK = scale dS^T Q.
// The reference runs one CTA per query row and adds dK/dV with fp32 atomics
// (nondeterministic).  Here the work is key-parallel:
//   * one workgroup (4 wavefronts) owns 128 keys of one (b, kv head); each
//     wave owns 32 keys whose K and V rows stay in registers as B operands of
//     v_mfma_f32_32x32x16_bf16;
//   * it walks the query blocks (32 rows) of every q head of its GQA group;
//     Q and dO tiles are staged in LDS row-major and transposed;
//   * dK^T and dV^T accumulate in registers across the whole walk: no
//     atomics on dK/dV, deterministic, GQA reduction for free;
//   * dS (bf16) goes through LDS and the block's dQ contribution
//     (32 rows x D) is added to an fp32 workspace with one coalesced
//     hardware float atomic per element; a last kernel scales and rounds it.
//   * causal: query blocks entirely above the block's first key are skipped.
#include "common.h"

namespace {

constexpr int BN = 128;  // keys per workgroup
constexpr int BM = 32;   // query rows per iteration
constexpr int KPAD = 8;
constexpr int TPAD = 4;
constexpr float kLog2e = 1.4426950408889634f;

DEVI float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
DEVI bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }
DEVI f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// 4 rows x 8 columns (row-major, 4 x 16 bytes) -> 8 rows x 4 columns
// (8 x 8 bytes) of 16-bit elements.  out[j] is column j as (r0,r1 | r2,r3).
DEVI void transpose4x8(const u32x4 (&in)[4], u32x2 (&out)[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    out[2 * j] = u32x2{__builtin_amdgcn_perm(in[1][j], in[0][j], 0x05040100u),
                       __builtin_amdgcn_perm(in[3][j], in[2][j], 0x05040100u)};
    out[2 * j + 1] = u32x2{__builtin_amdgcn_perm(in[1][j], in[0][j], 0x07060302u),
                           __builtin_amdgcn_perm(in[3][j], in[2][j], 0x07060302u)};
  }
}

template <int D>
struct __attribute__((aligned(16))) BwdSmem {
  bf16 qs[BM][D + KPAD];     // Q tile, row-major  (A operand of S)
  bf16 dos[BM][D + KPAD];    // dO tile, row-major (A operand of dP)
  bf16 qts[D][BM + TPAD];    // Q tile transposed  (A operand of dK^T)
  bf16 dots[D][BM + TPAD];   // dO tile transposed (A operand of dV^T)
  bf16 dss[BM][BN + KPAD];   // dS tile, row-major (A operand of dQ)
  bf16 kts[D][BN + KPAD];    // K block transposed (B operand of dQ)
  float lse2[BM];            // LSE * log2(e); +inf for rows past nq
  float delta[BM];
};

// Delta = rowsum(O o dO) in fp32 and zero the fp32 dQ accumulator.
template <int D>
__device__ void bwd_pre(const bf16* __restrict__ o, const bf16* __restrict__ dout,
                        float* __restrict__ delta, float* __restrict__ dq_acc, long rows) {
  constexpr int TPR = D / 8;  // threads per row, 8 elements each
  const long row = (long)blockIdx.x * (256 / TPR) + threadIdx.x / TPR;
  const int c = threadIdx.x % TPR;
  float s = 0.0f;
  if (row < rows) {
    float a[8], bb[8];
    Vec16<bf16>::load(o + row * D + 8 * c, a);
    Vec16<bf16>::load(dout + row * D + 8 * c, bb);
#pragma unroll
    for (int j = 0; j < 8; ++j) s += a[j] * bb[j];
    f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
    *reinterpret_cast<f32x4*>(dq_acc + row * D + 8 * c) = z;
    *reinterpret_cast<f32x4*>(dq_acc + row * D + 8 * c + 4) = z;
  }
#pragma unroll
  for (int off = TPR / 2; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
  if (row < rows && c == 0) delta[row] = s;
}

template <int D, bool CAUSAL>
__device__ void fa2_bwd_bf16(const bf16* __restrict__ q, const bf16* __restrict__ k,
                             const bf16* __restrict__ v, const bf16* __restrict__ dout,
                             const float* __restrict__ lse, const float* __restrict__ delta,
                             float* __restrict__ dq_acc, bf16* __restrict__ dk,
                             bf16* __restrict__ dv, int nq, int nk, float scale, int hq, int hkv,
                             int num_n_blocks, int total_blocks) {
  constexpr int DC = D / 16;  // d-chunks of 16 (QK^T, dO V^T)
  constexpr int DT = D / 32;  // d-tiles of 32 (dK^T, dV^T, dQ)
  constexpr int CPR = D / 8;  // 16-byte chunks per row
  constexpr int TILE_PAIRS = (BM / 4) * CPR;  // (4-row, 8-col) blocks per Q (or dO) tile
  constexpr int KT_PAIRS = (BN / 4) * CPR;    // same for the K block
  __shared__ BwdSmem<D> sm;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;

  const int id = xcd_remap(blockIdx.x, total_blocks);
  const int kvh = id / num_n_blocks;  // b * hkv + hk
  const int nb = id - kvh * num_n_blocks;
  const int b = kvh / hkv, hk = kvh - b * hkv;
  const int group = hq / hkv;
  const int n0 = nb * BN;
  const int kw0 = n0 + 32 * wave;  // this wave's first key
  const int mykey = kw0 + l32;

  const bf16* kb = k + (long)kvh * nk * D;
  const bf16* vb = v + (long)kvh * nk * D;

  // ---- K, V rows of this lane's key -> registers (B operands) --------------
  bf16x8 kreg[DC], vreg[DC];
  {
    const bool ok = mykey < nk;
    const bf16* kp = kb + (long)(ok ? mykey : 0) * D + 8 * g;
    const bf16* vp = vb + (long)(ok ? mykey : 0) * D + 8 * g;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      kreg[c] = as_bf16x8(ok ? *reinterpret_cast<const u32x4*>(kp + 16 * c) : u32x4{0, 0, 0, 0});
      vreg[c] = as_bf16x8(ok ? *reinterpret_cast<const u32x4*>(vp + 16 * c) : u32x4{0, 0, 0, 0});
    }
  }
  // ---- K block transposed -> LDS (B operand of dQ = dS K) ------------------
  for (int p = tid; p < KT_PAIRS; p += 256) {
    const int dg = p % CPR, kg = p / CPR;
    u32x4 in[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int key = n0 + 4 * kg + r;
      in[r] = key < nk ? *reinterpret_cast<const u32x4*>(kb + (long)key * D + 8 * dg)
                       : u32x4{0, 0, 0, 0};
    }
    u32x2 out[8];
    transpose4x8(in, out);
#pragma unroll
    for (int j = 0; j < 8; ++j) *reinterpret_cast<u32x2*>(&sm.kts[8 * dg + j][4 * kg]) = out[j];
  }

  // ---- query-block walk ------------------------------------------------------
  const int qb_first = CAUSAL ? n0 / BM : 0;
  const int n_qb = (nq + BM - 1) / BM;
  const int iters_per_head = n_qb > qb_first ? n_qb - qb_first : 0;
  const int n_iter = group * iters_per_head;

  // Staging: threads [0, TILE_PAIRS) carry Q, [TILE_PAIRS, 2*TILE_PAIRS) carry dO.
  const bool stager = tid < 2 * TILE_PAIRS;
  const bool st_is_do = tid >= TILE_PAIRS;
  const int st_p = st_is_do ? tid - TILE_PAIRS : tid;
  const int st_dg = st_p % CPR, st_rg = st_p / CPR;
  u32x4 stage[4];
  float st_lse = 0.0f, st_delta = 0.0f;

  auto head_of = [&](int it) { return it / iters_per_head; };
  auto qblock_of = [&](int it) { return qb_first + it % iters_per_head; };

  auto load_tile = [&](int it) {
    const long bh = (long)b * hq + (long)hk * group + head_of(it);
    const int qb0 = qblock_of(it) * BM;
    if (stager) {
      const bf16* src = st_is_do ? dout : q;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        int row = qb0 + 4 * st_rg + r;
        stage[r] = row < nq
                       ? *reinterpret_cast<const u32x4*>(src + (bh * nq + row) * D + 8 * st_dg)
                       : u32x4{0, 0, 0, 0};
      }
    }
    if (tid >= 192 && tid < 192 + BM) {
      int row = qb0 + (tid - 192);
      st_lse = row < nq ? lse[bh * nq + row] * kLog2e : INFINITY;
      st_delta = row < nq ? delta[bh * nq + row] : 0.0f;
    }
  };
  auto store_tile = [&]() {
    if (stager) {
      bf16(*rm)[D + KPAD] = st_is_do ? sm.dos : sm.qs;
      bf16(*tr)[BM + TPAD] = st_is_do ? sm.dots : sm.qts;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        *reinterpret_cast<u32x4*>(&rm[4 * st_rg + r][8 * st_dg]) = stage[r];
      u32x2 out[8];
      transpose4x8(stage, out);
#pragma unroll
      for (int j = 0; j < 8; ++j) *reinterpret_cast<u32x2*>(&tr[8 * st_dg + j][4 * st_rg]) = out[j];
    }
    if (tid >= 192 && tid < 192 + BM) {
      sm.lse2[tid - 192] = st_lse;
      sm.delta[tid - 192] = st_delta;
    }
  };

  f32x16 dk_acc[DT], dv_acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    dk_acc[t] = f32x16{};
    dv_acc[t] = f32x16{};
  }
  const float sl2 = scale * kLog2e;

  if (n_iter > 0) {
    load_tile(0);
    store_tile();
  }
  __syncthreads();

  for (int it = 0; it < n_iter; ++it) {
    const long bh = (long)b * hq + (long)hk * group + head_of(it);
    const int qb0 = qblock_of(it) * BM;
    if (it + 1 < n_iter) load_tile(it + 1);

    const bool wave_active = !(CAUSAL && kw0 > qb0 + BM - 1) && kw0 < nk;
    const bool need_mask = (kw0 + 32 > nk) || (CAUSAL && kw0 + 31 > qb0);
    uint32_t pb[8], dsb[8];
    if (wave_active) {
      // S = Q K^T and dP = dO V^T, C layout: lane = key (col), 16 query rows.
      f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        u32x4 aq = *reinterpret_cast<const u32x4*>(&sm.qs[l32][16 * c + 8 * g]);
        s = mfma32(as_bf16x8(aq), kreg[c], s);
      }
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        u32x4 ad = *reinterpret_cast<const u32x4*>(&sm.dos[l32][16 * c + 8 * g]);
        dp = mfma32(as_bf16x8(ad), vreg[c], dp);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r0 = 8 * j + 4 * g;  // first of this register group's 4 rows
        f32x4 l4 = *reinterpret_cast<const f32x4*>(&sm.lse2[r0]);
        f32x4 d4 = *reinterpret_cast<const f32x4*>(&sm.delta[r0]);
        float p[4], ds[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float pv = fast_exp2(s[4 * j + i] * sl2 - l4[i]);
          if (need_mask) {
            int qrow = qb0 + r0 + i;
            if (mykey >= nk || (CAUSAL && mykey > qrow)) pv = 0.0f;
          }
          p[i] = pv;
          ds[i] = pv * (dp[4 * j + i] - d4[i]);
        }
        pb[2 * j] = pack_bf16x2(p[0], p[1]);
        pb[2 * j + 1] = pack_bf16x2(p[2], p[3]);
        dsb[2 * j] = pack_bf16x2(ds[0], ds[1]);
        dsb[2 * j + 1] = pack_bf16x2(ds[2], ds[3]);
      }
      // dV^T += dO^T P and dK^T += Q^T dS (keys = columns, queries summed).
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        bf16x8 bp = as_bf16x8(u32x4{pb[4 * hh], pb[4 * hh + 1], pb[4 * hh + 2], pb[4 * hh + 3]});
        bf16x8 bs =
            as_bf16x8(u32x4{dsb[4 * hh], dsb[4 * hh + 1], dsb[4 * hh + 2], dsb[4 * hh + 3]});
#pragma unroll
        for (int t = 0; t < DT; ++t) {
          const bf16* dor = &sm.dots[32 * t + l32][16 * hh + 4 * g];
          u32x2 a0 = *reinterpret_cast<const u32x2*>(dor);
          u32x2 a1 = *reinterpret_cast<const u32x2*>(dor + 8);
          dv_acc[t] = mfma32(as_bf16x8(u32x4{a0[0], a0[1], a1[0], a1[1]}), bp, dv_acc[t]);
          const bf16* qr = &sm.qts[32 * t + l32][16 * hh + 4 * g];
          u32x2 c0 = *reinterpret_cast<const u32x2*>(qr);
          u32x2 c1 = *reinterpret_cast<const u32x2*>(qr + 8);
          dk_acc[t] = mfma32(as_bf16x8(u32x4{c0[0], c0[1], c1[0], c1[1]}), bs, dk_acc[t]);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) dsb[j] = 0u;
    }
    // dS -> LDS as [query][key] for the dQ product.
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t w = dsb[2 * j + (i >> 1)];
        uint16_t hbits = (i & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xffffu);
        reinterpret_cast<uint16_t*>(&sm.dss[8 * j + 4 * g + i][0])[32 * wave + l32] = hbits;
      }
    __syncthreads();
    // dQ[32 rows, d-tile = wave] += dS[32 x 128] K[128 x 32]
    if (wave < DT) {
      f32x16 acc = f32x16{};
#pragma unroll
      for (int c = 0; c < BN / 16; ++c) {
        u32x4 a = *reinterpret_cast<const u32x4*>(&sm.dss[l32][16 * c + 8 * g]);
        u32x4 bk = *reinterpret_cast<const u32x4*>(&sm.kts[32 * wave + l32][16 * c + 8 * g]);
        acc = mfma32(as_bf16x8(a), as_bf16x8(bk), acc);
      }
      float* dqb = dq_acc + (bh * nq) * D + 32 * wave + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        int row = qb0 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (row < nq) unsafeAtomicAdd(dqb + (long)row * D, acc[r]);
      }
    }
    __syncthreads();
    if (it + 1 < n_iter) store_tile();
    __syncthreads();
  }

  // ---- dK = scale * dK^T, dV = dV^T, lane = key, 16 d values per tile -------
  if (mykey < nk) {
    bf16* dkr = dk + ((long)kvh * nk + mykey) * D;
    bf16* dvr = dv + ((long)kvh * nk + mykey) * D;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        int d = 32 * t + 8 * j + 4 * g;
        *reinterpret_cast<u32x2*>(dkr + d) =
            u32x2{pack_bf16x2(dk_acc[t][4 * j] * scale, dk_acc[t][4 * j + 1] * scale),
                  pack_bf16x2(dk_acc[t][4 * j + 2] * scale, dk_acc[t][4 * j + 3] * scale)};
        *reinterpret_cast<u32x2*>(dvr + d) =
            u32x2{pack_bf16x2(dv_acc[t][4 * j], dv_acc[t][4 * j + 1]),
                  pack_bf16x2(dv_acc[t][4 * j + 2], dv_acc[t][4 * j + 3])};
      }
  }
}

// dq = bf16(scale * dq_acc)
__device__ void dq_convert(const float* __restrict__ acc, bf16* __restrict__ dq, float scale,
                           long n8) {
  long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  float a[8];
  f32x4 lo = *reinterpret_cast<const f32x4*>(acc + 8 * i);
  f32x4 hi = *reinterpret_cast<const f32x4*>(acc + 8 * i + 4);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    a[j] = lo[j] * scale;
    a[4 + j] = hi[j] * scale;
  }
  Vec16<bf16>::store(dq + 8 * i, a);
}

}  // namespace

extern "C" __global__ __launch_bounds__(256) void teeny_fa2_bwd_dq_convert_bf16(
    const float* acc, bf16* dq, float scale, long n8) {
  dq_convert(acc, dq, scale, n8);
}

#define TEENY_FA2_BWD_BF16_INST(D)                                                              \
  extern "C" __global__ __launch_bounds__(256) void teeny_fa2_bwd_pre_bf16_d##D(               \
      const bf16* o, const bf16* dout, float* delta, float* dq_acc, long rows) {               \
    bwd_pre<D>(o, dout, delta, dq_acc, rows);                                                   \
  }                                                                                             \
  extern "C" __global__ __launch_bounds__(256) void teeny_fa2_bwd_bf16_d##D##_c(               \
      const bf16* q, const bf16* k, const bf16* v, const bf16* dout, const float* lse,          \
      const float* delta, float* dq_acc, bf16* dk, bf16* dv, int nq, int nk, float scale,       \
      int hq, int hkv, int nnb, int total) {                                                    \
    fa2_bwd_bf16<D, true>(q, k, v, dout, lse, delta, dq_acc, dk, dv, nq, nk, scale, hq, hkv,   \
                          nnb, total);                                                          \
  }                                                                                             \
  extern "C" __global__ __launch_bounds__(256) void teeny_fa2_bwd_bf16_d##D##_n(               \
      const bf16* q, const bf16* k, const bf16* v, const bf16* dout, const float* lse,          \
      const float* delta, float* dq_acc, bf16* dk, bf16* dv, int nq, int nk, float scale,       \
      int hq, int hkv, int nnb, int total) {                                                    \
    fa2_bwd_bf16<D, false>(q, k, v, dout, lse, delta, dq_acc, dk, dv, nq, nk, scale, hq, hkv,  \
                           nnb, total);                                                         \
  }

TEENY_FA2_BWD_BF16_INST(64)
TEENY_FA2_BWD_BF16_INST(128)

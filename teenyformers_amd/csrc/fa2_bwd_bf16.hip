// bf16 flash-attention 2 backward on CDNA4 matrix cores (gfx950).
//
// Reference semantics: flash_attn2_causal_bwd (src/kernels/flash_attn2.rs:135-203)
// and flash_attn2_backward (:209-279):
//   P = exp(scale * Q K^T - LSE), dV = P^T dO, dP = dO V^T,
//   dS = P o (dP - Delta) with Delta = rowsum(O o dO), dQ = scale dS K,
//   dK = scale dS^T Q.
// The reference runs one CTA per query row and adds dK/dV with fp32 atomics
// (nondeterministic).  Here the backward is two kernels, both deterministic
// and free of atomics, launched dQ first:
//   1. dQ, query-parallel, shaped like the forward: each wave's Q and dO
//      rows are B operands in registers, 64-key tiles of K and V stream
//      through LDS (K^T via the transpose read), S^T and dP^T put one query
//      row in each lane, and dQ^T += K^T dS^T accumulates in registers.  Its
//      prologue forms Delta = rowsum(O o dO) for its rows in fp32 and writes
//      LSE * log2(e) and Delta per block of 32 rows for the next kernel (rows
//      past nq: +inf and 0, so the padded rows contribute P = 0);
//   2. dK/dV, key-parallel: one workgroup (4 wavefronts) owns 128 keys of one
//      (b, kv head); each wave's 32 K rows stay in registers and the block's
//      V rows in LDS as B operands of v_mfma_f32_32x32x16_bf16, and it walks
//      the 32-row query blocks of every q head of its GQA group (Q, dO tiles
//      streamed into double-buffered LDS by buffer_load ... lds and read both
//      row-wise and, through the LDS transpose read, as Q^T / dO^T),
//      accumulating dK^T and dV^T in registers: the GQA reduction comes for
//      free.  With few key blocks (long context, one sequence) the group's q
//      heads are split over 2-4 workgroups whose fp32 partial sums a third
//      kernel adds in a fixed order.
// Recomputing S and dP in the dQ kernel costs 7 matrix products per tile
// pair instead of 5; in exchange neither kernel needs dS round trips through
// LDS, fp32 atomics or a dQ accumulator in HBM (fp32 atomic adds of that dQ
// accumulation would cost more on MI355X than the recomputation they save).
// Causal: blocks entirely above the diagonal are skipped, diagonal blocks
// are masked.
#include "cdna4.h"

#include <type_traits>

namespace {

constexpr int BN = 128;  // keys per workgroup
constexpr int BM = 32;   // query rows per iteration; also the row block of the LSE / Delta array
constexpr float kLog2e = 1.4426950408889634f;

// four consecutive gradient values: bf16 (rounded to nearest even) or fp32
__device__ inline void store4(bf16* p, float a, float b, float c, float d) {
  *reinterpret_cast<u32x2*>(p) = u32x2{pack_bf16x2(a, b), pack_bf16x2(c, d)};
}
__device__ inline void store4(float* p, float a, float b, float c, float d) {
  *reinterpret_cast<f32x4*>(p) = f32x4{a, b, c, d};
}


// Per (b, q head) and block of BM query rows, ld holds BM values of
// -LSE / scale followed by BM values of -Delta (Delta = rowsum(O o dO)),
// fp32; rows past nq hold -inf and 0.  The dQ kernel writes it, the dK/dV
// kernel starts its score and dP accumulators from them, so that
// S' = S - LSE / scale gives P = exp2(scale log2(e) S') and dP' = dP - Delta
// gives dS = P dP' with no per-row value read while the products run.

// ===========================================================================
// dK / dV (key-parallel)
// ===========================================================================
template <int D>
struct __attribute__((aligned(16))) DkdvSmem {
  char v[BN * D * 2];     // the block's V rows: B operand of dP
  char q[2][BM * D * 2];  // Q tile: A operand of S, transposed A operand of dK^T
  char d[2][BM * D * 2];  // dO tile: A operand of dP, transposed A operand of dV^T
  float ld[2][2 * BM];    // LSE * log2(e) and Delta of the tile's rows
};

// hsplit > 1: the q heads of a GQA group are split over hsplit workgroups
// (more workgroups when few key blocks would leave CUs idle behind the
// heaviest causal block); each writes its fp32 dK^T, dV^T sums to
// part[2][hsplit][B * Hkv][nk][D] (dK unscaled), merged by fa2_dkdv_merge.
// NG = 2: the workgroup is two groups of 4 wavefronts (GRP 0 and 1, the
// kernel branches once on it) on the same 128 keys, each walking half of
// the workgroup's q heads in its own copy of the LDS block (smg[GRP]; a
// compile-time copy, so every LDS address keeps its immediate offset); at
// the end group 1's sums are added to group 0's through LDS, which stores.
template <int D, bool CAUSAL, typename GT, int NG = 1, int GRP = 0>
__device__ __forceinline__ void fa2_bwd_dkdv(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const bf16* __restrict__ dout, const float* __restrict__ ld, GT* __restrict__ dk,
    GT* __restrict__ dv, int nq, int nk, float scale, int hq, int hkv, int num_n_blocks,
    int total_blocks, int hsplit, float* __restrict__ part, int cu_pairs, DkdvSmem<D>* smg) {
  constexpr int DC = D / 16;            // d-chunks of 16 (QK^T, dO V^T)
  constexpr int DT = D / 32;            // d-tiles of 32 (dK^T, dV^T)
  constexpr int CPR = D / 8;            // 16-byte chunks per row
  constexpr int TCH = BM * CPR / 256;   // chunks per thread of a Q or dO tile
  constexpr int VCH = BN * CPR / 256;   // chunks per thread of the V block
  DkdvSmem<D>& sm = smg[GRP];

  // fp32 gradients: P and dS also enter the products as a second, low bf16
  // part (x = hi + lo, hi = bf16(x), lo = bf16(x - hi)), so their bf16
  // operand rounding (2^-9 relative) drops to 2^-17
  constexpr bool PRECISE = std::is_same<GT, float>::value;
  const int tid = NG == 1 ? (int)threadIdx.x : (int)threadIdx.x & 255;  // within the group
  // wave-uniform (an SGPR): every branch on it is a scalar branch
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;

  const int id = xcd_remap(blockIdx.x, total_blocks);
  int hh, nb;  // hh = (b * hkv + hk) * hsplit + hs; key block 0 sees the most query rows
  if (cu_pairs) {
    // every workgroup resident at once, two per CU (the host checks the
    // count and that each XCD's share holds whole heads and an even number
    // of key blocks): an XCD's i-th and (i + half)-th workgroups were
    // measured to share a CU, so the first half takes key blocks 0 ..
    // nnb/2 - 1 and the second half the rest in reverse, pairing block r
    // with block nnb - 1 - r and giving every CU about the same causal work
    const int per_x = total_blocks / TEENY_NUM_XCD, hpx = per_x / num_n_blocks;
    const int half = per_x / 2, x = id / per_x, L = id - x * per_x;
    const int lp = L < half ? L : L - half;
    hh = x * hpx + lp % hpx;
    nb = L < half ? lp / hpx : num_n_blocks - 1 - lp / hpx;
  } else {
    pair_order(id, num_n_blocks, total_blocks / num_n_blocks, hh, nb);
  }
  const int kvh = hh / hsplit, hs = hh - kvh * hsplit;
  const int b = kvh / hkv, hk = kvh - b * hkv;
  const int group = hq / hkv / hsplit / NG;  // q heads walked by this wavefront group
  const int head0 = hk * (hq / hkv) + (hs * NG + GRP) * group;
  const int n0 = nb * BN;
  const int kw0 = n0 + 32 * wave;  // this wave's first key
  const int mykey = kw0 + l32;
  const int nq_pad = (nq + BM - 1) / BM * BM;

  const bf16* kb = k + (long)kvh * nk * D;
  const bf16* vb = v + (long)kvh * nk * D;

  // ---- K row of this lane's key -> registers (B operand of S); keys past nk
  //      load key nk - 1 (computed, never stored) --------------------------
  bf16x8 kreg[DC];
  {
    const bf16* kp = kb + (long)min(mykey, nk - 1) * D + 8 * g;
#pragma unroll
    for (int c = 0; c < DC; ++c) kreg[c] = as_bf16x8(*reinterpret_cast<const u32x4*>(kp + 16 * c));
  }
  // ---- the block's V rows -> LDS (SWZ_DUAL; keys past nk re-read key nk-1) ----
  {
    const auto vr = make_rsrc(vb, nk * D * 2);
#pragma unroll
    for (int i = 0; i < VCH; ++i) {
      const int L = swz<SWZ_DUAL, D>(i * 256 + tid);  // the chunk this lane's slot holds
      const int key = min(n0 + L / CPR, nk - 1);
      dma16(vr, sm.v + i * 4096 + wave * 1024, key * D * 2 + (L % CPR) * 16, 0);
    }
  }

  // ---- query-block walk: (head, q-block) for every q head of the group ----
  const int qb_first = CAUSAL ? n0 / BM : 0;
  const int n_qb = nq_pad / BM;
  const int per_head = n_qb > qb_first ? n_qb - qb_first : 0;
  const int n_iter = group * per_head;

  // Q / dO tiles: chunk P = i*256 + tid of a tile holds tile chunk swz(P);
  // the swizzle repeats every 256 chunks.  Wave 0 also brings the rows'
  // LSE / Delta (2*BM floats, one dword per lane).  The descriptors cover a
  // whole head (rebuilt only when the walk moves to the next head) and the
  // tile's first row is the scalar offset; rows past nq lie outside the
  // range and load as zeros (their LSE is +inf and their dO zero, so P and
  // dS vanish).
  const uint32_t src = swz<SWZ_DUAL, D>(tid) * 16;
  int lhead = -1;
  __amdgpu_buffer_rsrc_t qr, dr, lr;
  auto load_tile = [&](int head, int qb, int buf) {
    if (head != lhead) {
      const long bh = (long)b * hq + head0 + head;
      qr = make_rsrc(q + bh * nq * D, nq * D * 2);
      dr = make_rsrc(dout + bh * nq * D, nq * D * 2);
      lr = make_rsrc(ld + bh * nq_pad * 2, nq_pad * 2 * 4);
      lhead = head;
    }
    const int row0 = qb * BM;
    char* qdst = sm.q[buf] + wave * 1024;
    char* ddst = sm.d[buf] + wave * 1024;
#pragma unroll
    for (int i = 0; i < TCH; ++i) {
      dma16(qr, qdst + i * 4096, src + i * 4096, row0 * D * 2);
      dma16(dr, ddst + i * 4096, src + i * 4096, row0 * D * 2);
    }
    if (wave == 0) {
      // the lane offset formed here (volatile: not hoisted out of the walk):
      // a value kept across the walk for this one load was spilled, and its
      // reload waited for every load in flight
      int ln;
      asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(lr, (lds_void*)sm.ld[buf], 4, ln * 4,
                                               row0 * 2 * 4, 0, 0);
    }
  };

  // ---- LDS read offsets (bytes) --------------------------------------------
  // rows: lane reads row l32 (V: 32*wave + l32), column chunk 2c + g
  int row_off[DC];
#pragma unroll
  for (int c = 0; c < DC; ++c) row_off[c] = swz<SWZ_DUAL, D>(l32 * CPR + 2 * c + g) * 16;
  const char* vrows = sm.v + wave * 32 * D * 2;  // the swizzle repeats every 16 rows
  // transposes (Q^T, dO^T): lane p of 16-lane group G reads row 8e + 4g + p/4
  // (+16 hh) and 8 bytes at column 32t + 16(G%2) + 4(p%4)
  int tr_off[DT][2];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int row = 8 * e + 4 * g + ((lane & 15) >> 2);
      const int col = 32 * t + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
      tr_off[t][e] = swz<SWZ_DUAL, D>(row * CPR + col / 8) * 16 + (col % 8) * 2;
    }
  auto tr_read = [&](const char* tile, int hh, int t) {
    const char* p = tile + hh * 16 * D * 2;
    u32x2 a0 = lds_read_tr(p + tr_off[t][0]), a1 = lds_read_tr(p + tr_off[t][1]);
    return as_bf16x8(u32x4{a0[0], a0[1], a1[0], a1[1]});
  };

  f32x16 dk_acc[DT], dv_acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    dk_acc[t] = f32x16{};
    dv_acc[t] = f32x16{};
  }
  const float sl2 = scale * kLog2e;

  int head = 0, qb = qb_first;  // (head, q-block) of the tile in buffer `it & 1`
  if (n_iter > 0) load_tile(0, qb_first, 0);
  __builtin_amdgcn_s_waitcnt(0);  // V block and the first tile
  __syncthreads();

  // one Q/dO tile; its buffer `buf` (= it % 2) is a constant in each of the
  // two unrolled steps, so every LDS address is a lane offset plus an
  // immediate
  for (int it = 0; it < n_iter; ++it) {
    const int buf = it & 1;
    const int qb0 = qb * BM;
    int nhead = head, nqb = qb + 1;
    if (nqb == n_qb) {
      nqb = qb_first;
      ++nhead;
    }
    const char* qt = sm.q[buf];
    const char* dt = sm.d[buf];
    const float* lt = sm.ld[buf];

    // The row values of this lane's 16 query rows (row 8 j + 4 g + i for
    // accumulator element 4 j + i) seed the score accumulator (-LSE / scale)
    // and the dP accumulator (-Delta).
    auto row_vals = [&](const float* p) {
      const f32x4 c0 = *reinterpret_cast<const f32x4*>(p + 4 * g);
      const f32x4 c1 = *reinterpret_cast<const f32x4*>(p + 8 + 4 * g);
      const f32x4 c2 = *reinterpret_cast<const f32x4*>(p + 16 + 4 * g);
      const f32x4 c3 = *reinterpret_cast<const f32x4*>(p + 24 + 4 * g);
      return f32x16{c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3],
                    c2[0], c2[1], c2[2], c2[3], c3[0], c3[1], c3[2], c3[3]};
    };
    // ---- S' = Q K^T - LSE / scale (lane = key, 16 query rows); Q rows read
    //      KPF products ahead ----
    constexpr int KPF = 2;
    f32x16 s, dp;
    {
      u32x4 aq[DC];
#pragma unroll
      for (int c = 0; c < KPF; ++c) aq[c] = *reinterpret_cast<const u32x4*>(qt + row_off[c]);
      s = row_vals(lt);
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        if (c + KPF < DC) aq[c + KPF] = *reinterpret_cast<const u32x4*>(qt + row_off[c + KPF]);
        s = mfma32(as_bf16x8(aq[c]), kreg[c], s);
      }
      sched_group(kDsRead, KPF + 4);
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        if (c + KPF < DC) sched_group(kDsRead, 1);
        sched_group(kMfma, 1);
      }
    }
    if (it + 1 < n_iter) load_tile(nhead, nqb, buf ^ 1);  // after the S products
    // ---- masking (boundary blocks only): scores -> -inf, so P = dS = 0 ----
    if ((kw0 + 32 > nk) || (CAUSAL && kw0 + 31 > qb0)) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int qrow = qb0 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (mykey >= nk || (CAUSAL && mykey > qrow)) s[r] = -INFINITY;
      }
    }
    // ---- dP' = dO V^T - Delta on the matrix cores, P = exp2(S' log2e
    //      scale) on the VALU; issue order fenced ----
    uint32_t pb[8], dsb[8];
    {
      constexpr int PPC = 8 / DC;  // P pairs per product
      constexpr int DPF = 2;       // dO / V rows read this many products ahead
      u32x4 ad[DC], av[DC];
#pragma unroll
      for (int c = 0; c < DPF; ++c) {
        ad[c] = *reinterpret_cast<const u32x4*>(dt + row_off[c]);
        av[c] = *reinterpret_cast<const u32x4*>(vrows + row_off[c]);
      }
      dp = row_vals(lt + BM);
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        if (c + DPF < DC) {
          ad[c + DPF] = *reinterpret_cast<const u32x4*>(dt + row_off[c + DPF]);
          av[c + DPF] = *reinterpret_cast<const u32x4*>(vrows + row_off[c + DPF]);
        }
        dp = mfma32(as_bf16x8(ad[c]), as_bf16x8(av[c]), dp);
#pragma unroll
        for (int i = 0; i < PPC; ++i) {
          const int r = 2 * (c * PPC + i);
          const float p0 = fast_exp2(s[r] * sl2);
          const float p1 = fast_exp2(s[r + 1] * sl2);
          s[r] = p0;
          s[r + 1] = p1;
          pb[r >> 1] = pack_bf16x2(p0, p1);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // ---- dV^T += dO^T P on the matrix cores, dS = P dP' on the VALU (hh = 0
    //      pairs after the first product, hh = 1 after ...); then
    //      dK^T += Q^T dS.  Transposed fragments read TPF products ahead ----
    {
      constexpr int NJ = 2 * DT;   // products of dV^T
      constexpr int PPJ = 8 / NJ;  // dS pairs per product
      constexpr int TPF = 2;
      bf16x8 ta[NJ];
      uint32_t plo[4], dslo[PRECISE ? 8 : 1];
#pragma unroll
      for (int j = 0; j < TPF; ++j) ta[j] = tr_read(dt, j / DT, j % DT);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int hh = j / DT, t = j % DT;
        if (j + TPF < NJ) ta[j + TPF] = tr_read(dt, (j + TPF) / DT, (j + TPF) % DT);
        dv_acc[t] = mfma32(ta[j], as_bf16x8(u32x4{pb[4 * hh], pb[4 * hh + 1], pb[4 * hh + 2],
                                                    pb[4 * hh + 3]}), dv_acc[t]);
        if constexpr (PRECISE) {
          if (t == 0)  // the low parts of this half's P (fp32 P is still in s)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              plo[i] = pack_bf16x2(s[8 * hh + 2 * i] - bf16lo(pb[4 * hh + i]),
                                   s[8 * hh + 2 * i + 1] - bf16hi(pb[4 * hh + i]));
          dv_acc[t] = mfma32(ta[j], as_bf16x8(u32x4{plo[0], plo[1], plo[2], plo[3]}), dv_acc[t]);
        }
#pragma unroll
        for (int i = 0; i < PPJ; ++i) {
          const int r = 2 * (j * PPJ + i);
          if constexpr (PRECISE) {
            const float ds0 = s[r] * dp[r];
            const float ds1 = s[r + 1] * dp[r + 1];
            dsb[r >> 1] = pack_bf16x2(ds0, ds1);
            dslo[r >> 1] = pack_bf16x2(ds0 - bf16lo(dsb[r >> 1]), ds1 - bf16hi(dsb[r >> 1]));
          } else {
            dsb[r >> 1] = pack_bf16x2(s[r] * dp[r], s[r + 1] * dp[r + 1]);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int j = 0; j < TPF; ++j) ta[j] = tr_read(qt, j / DT, j % DT);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int hh = j / DT, t = j % DT;
        if (j + TPF < NJ) ta[j + TPF] = tr_read(qt, (j + TPF) / DT, (j + TPF) % DT);
        dk_acc[t] = mfma32(ta[j], as_bf16x8(u32x4{dsb[4 * hh], dsb[4 * hh + 1], dsb[4 * hh + 2],
                                                     dsb[4 * hh + 3]}), dk_acc[t]);
        if constexpr (PRECISE)
          dk_acc[t] = mfma32(ta[j], as_bf16x8(u32x4{dslo[4 * hh], dslo[4 * hh + 1], dslo[4 * hh + 2],
                                                       dslo[4 * hh + 3]}), dk_acc[t]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    head = nhead;
    qb = nqb;
    __builtin_amdgcn_s_waitcnt(0);  // this thread's loads of the next tile have landed
    __syncthreads();
  }

  if constexpr (NG == 2) {
    // group 1's sums into group 0's through LDS, dK^T then dV^T (16 bytes
    // per lane and step, consecutive lanes consecutive); the walk's last
    // barrier has retired every tile read
    f32x4* x = reinterpret_cast<f32x4*>(smg) + wave * DT * 4 * 64 + lane;
    auto exchange = [&](f32x16(&acc)[DT]) {
      if constexpr (GRP == 1)
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            x[(t * 4 + j) * 64] =
                f32x4{acc[t][4 * j], acc[t][4 * j + 1], acc[t][4 * j + 2], acc[t][4 * j + 3]};
      __syncthreads();
      if constexpr (GRP == 0)
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const f32x4 y = x[(t * 4 + j) * 64];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[t][4 * j + i] += y[i];
          }
      __syncthreads();
    };
    exchange(dk_acc);
    exchange(dv_acc);
    if constexpr (GRP == 1) return;
  }
  // ---- dK = scale * dK^T, dV = dV^T (rows = this wavefront's 32 keys),
  //      through LDS a whole row per store: no LDS read follows the walk's
  //      last barrier (or, with two groups, the exchange's), so each
  //      wavefront's area is free ----
  static_assert(sizeof(DkdvSmem<D>) >= 4 * 32 * D * sizeof(float), "tiles fit the LDS block");
  char* etile = reinterpret_cast<char*>(smg) + wave * (32 * D * (int)sizeof(float));
  if (hsplit > 1) {  // fp32 sums of this workgroup's heads
    const long n_kvh = total_blocks / num_n_blocks / hsplit;
    float* pk = part + (((long)hs * n_kvh + kvh) * nk + kw0) * D;
    float* pv = pk + (long)hsplit * n_kvh * nk * D;
    store_tile_rows<D, float>(etile, pk, nk - kw0, [&](int t, int j) {
      return f32x4{dk_acc[t][4 * j], dk_acc[t][4 * j + 1], dk_acc[t][4 * j + 2], dk_acc[t][4 * j + 3]};
    });
    store_tile_rows<D, float>(etile, pv, nk - kw0, [&](int t, int j) {
      return f32x4{dv_acc[t][4 * j], dv_acc[t][4 * j + 1], dv_acc[t][4 * j + 2], dv_acc[t][4 * j + 3]};
    });
    return;
  }
  store_tile_rows<D, GT>(etile, dk + ((long)kvh * nk + kw0) * D, nk - kw0, [&](int t, int j) {
    return f32x4{dk_acc[t][4 * j] * scale, dk_acc[t][4 * j + 1] * scale,
                 dk_acc[t][4 * j + 2] * scale, dk_acc[t][4 * j + 3] * scale};
  });
  store_tile_rows<D, GT>(etile, dv + ((long)kvh * nk + kw0) * D, nk - kw0, [&](int t, int j) {
    return f32x4{dv_acc[t][4 * j], dv_acc[t][4 * j + 1], dv_acc[t][4 * j + 2], dv_acc[t][4 * j + 3]};
  });
}

// dK = scale * sum of the hsplit partial dK^T, dV = sum of the dV^T, in
// split order; n = B * Hkv * nk * D (a multiple of 8), 8 values per thread.
template <typename GT>
__device__ void fa2_dkdv_merge(const float* __restrict__ part, GT* __restrict__ dk,
                               GT* __restrict__ dv, long n, int hsplit, float scale) {
  const long i = ((long)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i >= n) return;
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    const float* src = part + (long)w * hsplit * n + i;
    float acc[8];
    Vec16<float>::load(src, acc);
    Vec16<float>::load(src + 4, acc + 4);
    for (int s = 1; s < hsplit; ++s) {
      float a[8];
      Vec16<float>::load(src + (long)s * n, a);
      Vec16<float>::load(src + (long)s * n + 4, a + 4);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] += a[j];
    }
    if (w == 0)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] *= scale;
    GT* dst = (w == 0 ? dk : dv) + i;
    store4(dst, acc[0], acc[1], acc[2], acc[3]);
    store4(dst + 4, acc[4], acc[5], acc[6], acc[7]);
  }
}

// ===========================================================================
// dQ (query-parallel)
// ===========================================================================
constexpr int QBM = 128;  // query rows per workgroup (4 waves x 32)
constexpr int QBN = 64;   // keys per LDS tile, processed as two 32-key halves
constexpr int QKBUF = 3;  // K tiles: previous (its transpose is still read), current, loading
constexpr int QVBUF = 2;  // V tiles: current, loading

template <int D>
struct __attribute__((aligned(16))) DqSmem {
  char k[QKBUF][QBN * D * 2];
  char v[QVBUF][QBN * D * 2];
};

// PACK: GQA groups of 4 packed as in the forward, one workgroup per (b, kv
// head, 32 query rows), wavefront w on q head kv head * 4 + w
template <int D, bool CAUSAL, typename GT, bool PACK = false>
__device__ void fa2_bwd_dq(const bf16* __restrict__ q, const bf16* __restrict__ k,
                           const bf16* __restrict__ v, const bf16* __restrict__ o,
                           const bf16* __restrict__ dout, const float* __restrict__ lse,
                           float* __restrict__ ld, GT* __restrict__ dq, int nq, int nk,
                           float scale, int hq, int hkv, int num_m_blocks, int total_blocks) {
  constexpr int DC = D / 16;
  constexpr int DT = D / 32;
  constexpr int CPR = D / 8;
  constexpr int TILE = QBN * D * 2;    // bytes per tile
  constexpr int HALF = 32 * D * 2;     // bytes of 32 rows
  constexpr int TCH = QBN * CPR / 256; // 16-byte chunks per thread per tile
  __shared__ DqSmem<D> sm;

  // fp32 gradients: dS also enters the dQ product as a second, low bf16 part
  // (dS = hi + lo), so its bf16 operand rounding drops from 2^-9 to 2^-17
  constexpr bool PRECISE = std::is_same<GT, float>::value;
  const int tid = threadIdx.x;
  // wave-uniform (an SGPR): every branch on it is a scalar branch
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;

  const int id = xcd_remap(blockIdx.x, total_blocks);
  int bh, rank;
  pair_order(id, num_m_blocks, total_blocks / num_m_blocks, bh, rank);
  const int mb = num_m_blocks - 1 - rank;  // the last query block is the heaviest
  // bhq: this wavefront's (b, q head); wrow0: its first query row; blk_end:
  // one past the workgroup's last row
  int bhq, wrow0, blk_end;
  long kvh;
  if constexpr (PACK) {
    const int b = bh / hkv;
    kvh = bh;
    bhq = b * hq + (bh - b * hkv) * 4 + wave;
    wrow0 = mb * 32;
    blk_end = wrow0 + 32;
  } else {
    const int b = bh / hq, h = bh - b * hq;
    kvh = (long)b * hkv + h / (hq / hkv);
    bhq = bh;
    wrow0 = mb * QBM + wave * 32;
    blk_end = mb * QBM + QBM;
  }
  const int qrow = wrow0 + l32;
  const bool qok = qrow < nq;

  const bf16* kb = k + kvh * (long)nk * D;
  const bf16* vb = v + kvh * (long)nk * D;

  // ---- this lane's Q and dO row (B operands), LSE and Delta ----------------
  // rows past nq load row nq - 1 and get LSE = +inf (P = 0): never stored
  bf16x8 qreg[DC], doreg[DC];
  {
    const long row = (long)bhq * nq + min(qrow, nq - 1);
    const bf16* qp = q + row * D + 8 * g;
    const bf16* dp = dout + row * D + 8 * g;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      qreg[c] = as_bf16x8(*reinterpret_cast<const u32x4*>(qp + 16 * c));
      doreg[c] = as_bf16x8(*reinterpret_cast<const u32x4*>(dp + 16 * c));
    }
  }
  // LSE * log2(e) and Delta = rowsum(O o dO) of this row (rows past nq: +inf
  // and 0): the lane holds half of the row's d values (8 g + 16 c ..), the
  // other half is in lane l ^ 32.  For the dK/dV kernel, which runs after
  // this one, ld gets -LSE / scale and -Delta: the initial values of its
  // score and dP accumulators.
  float lse2 = INFINITY, dlt = 0.0f;
  {
    const long row = (long)bhq * nq + min(qrow, nq - 1);
    const bf16* op = o + row * D + 8 * g;
    float part = 0.0f;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      float a[8], bb[8];
      Vec16<bf16>::load(op + 16 * c, a);
      const u32x4 dw = __builtin_bit_cast(u32x4, doreg[c]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bb[2 * j] = bf16lo(dw[j]);
        bb[2 * j + 1] = bf16hi(dw[j]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) part += a[j] * bb[j];
    }
    part += other_half(part);
    if (qok) {
      lse2 = lse[(long)bhq * nq + qrow] * kLog2e;
      dlt = part;
    }
    const int nq_pad = (nq + BM - 1) / BM * BM;  // ld rows: whole blocks of BM
    if (g == 0 && qrow < nq_pad) {
      float* blk = ld + ((long)bhq * nq_pad + qrow) / BM * (2 * BM);
      blk[qrow % BM] = qok ? -lse[(long)bhq * nq + qrow] / scale : -INFINITY;
      blk[BM + qrow % BM] = -dlt;
    }
  }
  const float sl2 = scale * kLog2e;

  int kend = nk;
  if (CAUSAL) kend = min(nk, blk_end);
  const int n_iter = (kend + QBN - 1) / QBN;
  // causal: the workgroup's tiles past this wavefront's last row are fully
  // masked for it; it computes only the first n_live (wave-uniform)
  const int n_live = CAUSAL ? min(n_iter, (wrow0 + 31) / QBN + 1) : n_iter;

  // ---- K / V tiles: buffer_load ... lds, both SWZ_DUAL ----------------------
  const uint32_t src = swz<SWZ_DUAL, D>(wave * 64 + lane) * 16;
  const auto krsrc = make_rsrc(kb, nk * D * 2);
  const auto vrsrc = make_rsrc(vb, nk * D * 2);
  auto load_tile = [&](int it, int koff, int voff) {
    const int kbase = it * QBN;
    char* kdst = sm.k[0] + koff + wave * 64 * 16;
    char* vdst = sm.v[0] + voff + wave * 64 * 16;
    const int sbase = kbase * D * 2;
    if (kbase + QBN <= nk) {
#pragma unroll
      for (int i = 0; i < TCH; ++i) {
        dma16(krsrc, kdst + i * 4096, src, sbase + i * 4096);
        dma16(vrsrc, vdst + i * 4096, src, sbase + i * 4096);
      }
    } else {  // rows past the sequence re-read its last row (masked later)
      const int last = nk - 1 - kbase;
#pragma unroll
      for (int i = 0; i < TCH; ++i) {
        const int o = i * 4096 + src;
        const int oc = min(o / (2 * D), last) * (2 * D) + o % (2 * D);
        dma16(krsrc, kdst + i * 4096, oc, sbase);
        dma16(vrsrc, vdst + i * 4096, oc, sbase);
      }
    }
  };
  auto next_buf = [](int off, int n) { return off + TILE == n * TILE ? 0 : off + TILE; };

  // ---- LDS read offsets (bytes) --------------------------------------------
  // rows: lane reads row l32 (+32 per half), column chunk 2c + g
  int row_off[DC];
#pragma unroll
  for (int c = 0; c < DC; ++c) row_off[c] = swz<SWZ_DUAL, D>(l32 * CPR + 2 * c + g) * 16;
  // K^T (transpose reads): lane p of 16-lane group G reads row 8e + 4g + p/4
  // (+16 hh, +32 per half: the swizzle repeats every 16 rows) and 8 bytes at
  // column 32t + 16(G%2) + 4(p%4)
  int tr_off[DT][2];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int row = 8 * e + 4 * g + ((lane & 15) >> 2);
      const int col = 32 * t + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
      tr_off[t][e] = swz<SWZ_DUAL, D>(row * CPR + col / 8) * 16 + (col % 8) * 2;
    }

  f32x16 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f32x16{};
  // dS^T of the previous 32-key half (B operand of its delayed dQ^T product)
  uint32_t dsb_prev[8], dsb_new[8];
  constexpr int NLO = PRECISE ? 8 : 1;
  uint32_t dslo_prev[NLO], dslo_new[NLO];
#pragma unroll
  for (int i = 0; i < 8; ++i) dsb_prev[i] = 0;
#pragma unroll
  for (int i = 0; i < NLO; ++i) dslo_prev[i] = 0;

  // S^T = K Q^T and dP^T = V dO^T for 32 keys (lane = query row, 16 keys),
  // fragments read KPF steps ahead
  auto s_dp = [&](const char* kt, const char* vt, f32x16& s, f32x16& dp) {
    constexpr int KPF = 2;
    s = f32x16{};
    dp = f32x16{};
    u32x4 ak[DC], av[DC];
#pragma unroll
    for (int c = 0; c < KPF; ++c) {
      ak[c] = *reinterpret_cast<const u32x4*>(kt + row_off[c]);
      av[c] = *reinterpret_cast<const u32x4*>(vt + row_off[c]);
    }
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      if (c + KPF < DC) {
        ak[c + KPF] = *reinterpret_cast<const u32x4*>(kt + row_off[c + KPF]);
        av[c + KPF] = *reinterpret_cast<const u32x4*>(vt + row_off[c + KPF]);
      }
      s = mfma32(as_bf16x8(ak[c]), qreg[c], s);
      dp = mfma32(as_bf16x8(av[c]), doreg[c], dp);
    }
    sched_group(kDsRead, 2 * KPF);
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      if (c + KPF < DC) sched_group(kDsRead, 2);
      sched_group(kMfma, 2);
    }
  };
  // keys past nk or (causal) past the row -> score -inf, so P = dS = 0
  auto mask = [&](int kb0, f32x16& s) {
    if ((kb0 + 32 > nk) || (CAUSAL && kb0 + 31 > wrow0)) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb0 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (key >= nk || (CAUSAL && key > qrow)) s[r] = -INFINITY;
      }
    }
  };
  // dQ^T += K^T dS^T, product j = (hh, t): keys 16hh.. of a half, d-tile t
  constexpr int NJ = 2 * DT;
  auto dq_read = [&](const char* kt, int j) {
    const int t = j % DT, hh = j / DT;
    const char* p = kt + hh * 16 * D * 2;
    u32x2 a0 = lds_read_tr(p + tr_off[t][0]), a1 = lds_read_tr(p + tr_off[t][1]);
    return u32x4{a0[0], a0[1], a1[0], a1[1]};
  };
  auto dq_mfma = [&](int j, u32x4 a) {
    const int t = j % DT, hh = j / DT;
    bf16x8 bop = as_bf16x8(
        u32x4{dsb_prev[4 * hh], dsb_prev[4 * hh + 1], dsb_prev[4 * hh + 2], dsb_prev[4 * hh + 3]});
    acc[t] = mfma32(as_bf16x8(a), bop, acc[t]);
    if constexpr (PRECISE)
      acc[t] = mfma32(as_bf16x8(a),
                      as_bf16x8(u32x4{dslo_prev[4 * hh], dslo_prev[4 * hh + 1],
                                      dslo_prev[4 * hh + 2], dslo_prev[4 * hh + 3]}),
                      acc[t]);
  };
  // P and dS = P (dP - Delta) for score pair r, r+1 -> packed bf16
  auto ds_pair = [&](const f32x16& s, const f32x16& dp, int r) {
    const float p0 = fast_exp2(__builtin_fmaf(s[r], sl2, -lse2));
    const float p1 = fast_exp2(__builtin_fmaf(s[r + 1], sl2, -lse2));
    const float ds0 = p0 * (dp[r] - dlt), ds1 = p1 * (dp[r + 1] - dlt);
    dsb_new[r >> 1] = pack_bf16x2(ds0, ds1);
    if constexpr (PRECISE)
      dslo_new[r >> 1] = pack_bf16x2(ds0 - bf16lo(dsb_new[r >> 1]), ds1 - bf16hi(dsb_new[r >> 1]));
  };
  // the previous half's dQ^T product on the matrix cores, interleaved with
  // this half's exponentials on the VALU (issue order fenced)
  auto dq_and_ds = [&](const char* kprev, const f32x16& s, const f32x16& dp) {
    constexpr int VPF = 2;
    constexpr int PPJ = 8 / NJ;  // pairs per product
    u32x4 va[NJ];
#pragma unroll
    for (int j = 0; j < VPF; ++j) va[j] = dq_read(kprev, j);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (j + VPF < NJ) va[j + VPF] = dq_read(kprev, j + VPF);
      dq_mfma(j, va[j]);
#pragma unroll
      for (int i = 0; i < PPJ; ++i) ds_pair(s, dp, 2 * (j * PPJ + i));
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pin(dsb_new[i]);
      dsb_prev[i] = dsb_new[i];
    }
    if constexpr (PRECISE)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        pin(dslo_new[i]);
        dslo_prev[i] = dslo_new[i];
      }
  };

  // The first lagged product reads the K half "before" tile 0 with dS = 0:
  // zero it (buffer QKBUF-1, second half) so that 0 * K stays 0.
  for (int i = tid; i < HALF / 16; i += 256)
    *reinterpret_cast<u32x4*>(sm.k[QKBUF - 1] + HALF + 16 * i) = u32x4{0, 0, 0, 0};
  // tile 1 is requested with tile 0, before the first wait (its latency
  // overlaps tile 0's); the barrier alone, since __syncthreads would wait
  // for tile 1's loads too
  if (n_iter > 0) load_tile(0, 0, 0);
  if (n_iter > 1) {
    load_tile(1, TILE, TILE);
    __builtin_amdgcn_s_waitcnt(kVmWaitLgkm0<2 * TCH>());
  } else {
    __builtin_amdgcn_s_waitcnt(0);
  }
  barrier_only();

  // Tile it uses K buffer it % 3 and V buffer it % 2.  The loop is unrolled
  // over the 6 tiles after which both rotations repeat, so every LDS address
  // is a lane offset plus a constant (the read's immediate offset) instead of
  // one address add per read.
  auto tile_step = [&](int it, auto KB, auto VB) {
    constexpr int kb = decltype(KB)::value, vb = decltype(VB)::value;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      f32x16 s, dp;
      s_dp(sm.k[kb] + u * HALF, sm.v[vb] + u * HALF, s, dp);
      if (u == 0 && it > 0 && it + 1 < n_iter)  // after the first products (as in the forward)
        load_tile(it + 1, ((kb + 1) % QKBUF) * TILE, ((vb + 1) % QVBUF) * TILE);
      mask(it * QBN + 32 * u, s);
      // the pending dS^T is of the previous half: tile it-1's second half, then this tile's first
      dq_and_ds(u == 0 ? sm.k[(kb + QKBUF - 1) % QKBUF] + HALF : sm.k[kb], s, dp);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this thread's loads of tile it+1 have landed
    __syncthreads();
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  int it = 0;
  for (; it + 6 <= n_live; it += 6) {
    tile_step(it, I0{}, I0{});
    tile_step(it + 1, I1{}, I1{});
    tile_step(it + 2, I2{}, I0{});
    tile_step(it + 3, I0{}, I1{});
    tile_step(it + 4, I1{}, I0{});
    tile_step(it + 5, I2{}, I1{});
  }
  // the last n_live % 6 tiles (same buffer sequence)
  if (it < n_live) tile_step(it, I0{}, I0{});
  if (it + 1 < n_live) tile_step(it + 1, I1{}, I1{});
  if (it + 2 < n_live) tile_step(it + 2, I2{}, I0{});
  if (it + 3 < n_live) tile_step(it + 3, I0{}, I1{});
  if (it + 4 < n_live) tile_step(it + 4, I1{}, I0{});
  if (n_iter > 0) {  // tile n_live-1's second half: its dS^T product is pending
    const char* kl = sm.k[0] + ((n_live - 1) % QKBUF) * TILE + HALF;
#pragma unroll
    for (int j = 0; j < NJ; ++j) dq_mfma(j, dq_read(kl, j));
    // a wavefront whose rows end before the workgroup's last tiles still
    // loads its share of them and meets the workgroup at each of their
    // barriers (tile t + 1 goes to K buffer (t + 1) % 3, V buffer (t + 1) % 2)
    for (int t = n_live; t < n_iter; ++t) {
      if (t + 1 < n_iter) load_tile(t + 1, ((t + 1) % QKBUF) * TILE, ((t + 1) % QVBUF) * TILE);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
  }

  // dQ rows through LDS (the K/V buffers: every wavefront's last product has
  // read them once all have passed this barrier), stored whole rows at a time
  static_assert(sizeof(DqSmem<D>) >= 4 * 32 * D * sizeof(GT), "dQ tiles fit the K/V buffers");
  __builtin_amdgcn_s_waitcnt(kVmWaitLgkm0<63>());
  barrier_only();
  (void)qok;
  store_tile_rows<D, GT>(reinterpret_cast<char*>(&sm) + wave * (32 * D * (int)sizeof(GT)),
                         dq + ((long)bhq * nq + wrow0) * D, nq - wrow0, [&](int t, int j) {
                           return f32x4{acc[t][4 * j] * scale, acc[t][4 * j + 1] * scale,
                                        acc[t][4 * j + 2] * scale, acc[t][4 * j + 3] * scale};
                         });
}

}  // namespace

// Kernels for D in {64, 128}, causal (_c) or not (_n); GT is the gradient
// type: bf16 (the inputs' type) or fp32 (suffix _g32, the accumulators
// stored unrounded).
#define TEENY_FA2_BWD_BF16_INST(D, CZ, CAUSAL, GT, SFX)                                          \
  extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))      \
  void teeny_fa2_bwd_dkdv_bf16_d##D##_##CZ##SFX(                                                \
      const bf16* q, const bf16* k, const bf16* v, const bf16* dout, const float* ld, GT* dk,   \
      GT* dv, int nq, int nk, float scale, int hq, int hkv, int nnb, int total, int hsplit,     \
      float* part, int cu_pairs) {                                                              \
    __shared__ DkdvSmem<D> sm[1];                                                               \
    fa2_bwd_dkdv<D, CAUSAL, GT>(q, k, v, dout, ld, dk, dv, nq, nk, scale, hq, hkv, nnb, total, \
                                hsplit, part, cu_pairs, sm);                                    \
  }                                                                                             \
  extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))      \
  void teeny_fa2_bwd_dq_bf16_d##D##_##CZ##SFX(                                                  \
      const bf16* q, const bf16* k, const bf16* v, const bf16* o, const bf16* dout,             \
      const float* lse, float* ld, GT* dq, int nq, int nk, float scale, int hq, int hkv,        \
      int nmb, int total) {                                                                     \
    fa2_bwd_dq<D, CAUSAL, GT>(q, k, v, o, dout, lse, ld, dq, nq, nk, scale, hq, hkv, nmb,      \
                              total);                                                           \
  }

TEENY_FA2_BWD_BF16_INST(64, c, true, bf16, )
TEENY_FA2_BWD_BF16_INST(64, n, false, bf16, )
TEENY_FA2_BWD_BF16_INST(128, c, true, bf16, )
TEENY_FA2_BWD_BF16_INST(128, n, false, bf16, )
TEENY_FA2_BWD_BF16_INST(64, c, true, float, _g32)
TEENY_FA2_BWD_BF16_INST(64, n, false, float, _g32)
TEENY_FA2_BWD_BF16_INST(128, c, true, float, _g32)
TEENY_FA2_BWD_BF16_INST(128, n, false, float, _g32)

// dK/dV of causal GQA with an even group, in two wavefront groups (512
// threads, one workgroup per CU)
#define TEENY_FA2_BWD_DKDV_HG2_INST(D, GT, SFX)                                                  \
  extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))      \
  void teeny_fa2_bwd_dkdv_bf16_d##D##_c_hg2##SFX(                                               \
      const bf16* q, const bf16* k, const bf16* v, const bf16* dout, const float* ld, GT* dk,   \
      GT* dv, int nq, int nk, float scale, int hq, int hkv, int nnb, int total, int hsplit,     \
      float* part, int cu_pairs) {                                                              \
    __shared__ DkdvSmem<D> sm[2];                                                               \
    if (threadIdx.x >= 256)                                                                     \
      fa2_bwd_dkdv<D, true, GT, 2, 1>(q, k, v, dout, ld, dk, dv, nq, nk, scale, hq, hkv, nnb,  \
                                      total, hsplit, part, cu_pairs, sm);                       \
    else                                                                                        \
      fa2_bwd_dkdv<D, true, GT, 2, 0>(q, k, v, dout, ld, dk, dv, nq, nk, scale, hq, hkv, nnb,  \
                                      total, hsplit, part, cu_pairs, sm);                       \
  }

TEENY_FA2_BWD_DKDV_HG2_INST(64, bf16, )
TEENY_FA2_BWD_DKDV_HG2_INST(128, bf16, )
TEENY_FA2_BWD_DKDV_HG2_INST(64, float, _g32)
TEENY_FA2_BWD_DKDV_HG2_INST(128, float, _g32)

// dQ of causal GQA groups of 4, packed (hq = 4 hkv)
#define TEENY_FA2_BWD_DQ_G4_INST(D, GT, SFX)                                                     \
  extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))      \
  void teeny_fa2_bwd_dq_bf16_d##D##_c_g4##SFX(                                                  \
      const bf16* q, const bf16* k, const bf16* v, const bf16* o, const bf16* dout,             \
      const float* lse, float* ld, GT* dq, int nq, int nk, float scale, int hq, int hkv,        \
      int nmb, int total) {                                                                     \
    fa2_bwd_dq<D, true, GT, true>(q, k, v, o, dout, lse, ld, dq, nq, nk, scale, hq, hkv, nmb,  \
                                  total);                                                       \
  }

TEENY_FA2_BWD_DQ_G4_INST(64, bf16, )
TEENY_FA2_BWD_DQ_G4_INST(128, bf16, )
TEENY_FA2_BWD_DQ_G4_INST(64, float, _g32)
TEENY_FA2_BWD_DQ_G4_INST(128, float, _g32)

extern "C" __global__ __launch_bounds__(256) void teeny_fa2_dkdv_merge_bf16(
    const float* part, bf16* dk, bf16* dv, long n, int hsplit, float scale) {
  fa2_dkdv_merge(part, dk, dv, n, hsplit, scale);
}
extern "C" __global__ __launch_bounds__(256) void teeny_fa2_dkdv_merge_bf16_g32(
    const float* part, float* dk, float* dv, long n, int hsplit, float scale) {
  fa2_dkdv_merge(part, dk, dv, n, hsplit, scale);
}

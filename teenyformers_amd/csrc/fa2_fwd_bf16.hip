// bf16 flash-attention 2 forward on CDNA4 matrix cores (gfx950).
//
// Reference semantics: flash_attn2_causal_fwd (src/kernels/flash_attn2.rs:61-126)
// and the bidirectional forward (:57-58): O = softmax(scale * Q K^T [+ causal
// mask k > q]) V per query row, LSE = m + ln(l) in the natural-log,
// scaled-score domain (:121-122).  The reference is fp32 with one CTA per
// query row; this kernel keeps bf16 operands with fp32 accumulation and a
// fp32 online softmax.
//
// Tiling (one workgroup = 4 wavefronts = 128 query rows of one (b, h); two
// or three workgroups per CU, so the waves on each SIMD run independently
// and cover each other's MFMA / VALU phases: the causal D = 128 forms take
// 32-key tiles, whose registers (168) and LDS (40 KiB) let three workgroups
// share a CU, the others 64-key tiles (three per CU at D = 64, two at
// D = 128).  Long GQA sequences take the _w8 form: 8 wavefronts = 256 rows
// share each K/V tile, one workgroup per CU, half the L2 -> LDS traffic per
// product):
//   * each wave owns 32 query rows; its Q rows live in registers as the
//     B operand of v_mfma_f32_32x32x16_bf16;
//   * K/V advance in tiles of 64 (or 32) keys that buffer_load ... lds streams into
//     LDS one tile ahead (K: 2 buffers, V: 3, since the PV product of a tile
//     runs one iteration late); K is stored SWZ_ROW and read row-wise as the
//     A operand of S^T = K Q^T, V is stored SWZ_DUAL and read with the LDS
//     transpose read ds_read_b64_tr_b16 as the A operand of O^T += V^T P^T
//     (both bank-conflict free);
//   * S^T puts one query row in each lane (lane % 32) and 16 keys per lane
//     per 32-key subtile, so the row max / row sum are in-lane plus one
//     exchange between the two lane halves;
//   * the fp32 accumulator of S^T, rounded to bf16, is already in the
//     B-operand layout of O^T += V^T P^T (keys are a summation index, so the
//     key order inside each 16-key chunk only has to agree between A and B);
//   * the PV product of tile i-1 is issued one MFMA at a time between the
//     row max and exponentials of tile i (fenced issue order), so the matrix
//     cores and the VALU work at once within one wave;
//   * online softmax in the log2 domain (exp2 with log2(e) folded into the
//     scale) without a per-tile maximum: the exponent offset is the row's
//     maximum over its first key tile, and a later tile's P = 2^(t - m) is
//     only checked afterwards through its row sums (any partial sum at or
//     above 2^31, or not finite, redoes the tile with its maximum and
//     rescales O and l); P, l and O stay far from fp32 overflow, and the
//     floating-point results are scale-invariant;
//   * causal: key tiles past the block's last row are not loaded, diagonal
//     tiles are masked;
//   * GQA: q head h reads kv head h / (Hq / Hkv);
//   * scheduling: block ids are remapped so one XCD works through whole heads
//     (K/V stay in that XCD's L2), heaviest causal blocks first;
//   * o_merged: O is stored [B, Sq, Hq * D] (MergeHeadsOp fused, rows Hq D
//     apart) instead of [B, Hq, Sq, D]; rope_cs: Q is read from the fused
//     QKV projection and rotated (RoPE) as it is loaded.
#include "cdna4.h"

#include <type_traits>

namespace {

constexpr int SUBN = 32;  // keys per subtile: one S^T accumulator of 32 keys x 32 rows
constexpr int KBUF = 2;  // K tiles in flight: read by QK(i), loading i+1
constexpr int VBUF = 3;  // V tiles: read by PV(i-1), waiting (i), loading (i+1)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kPmax = 2147483648.0f;  // 2^31: a tile's partial row sums stay below

template <int D, int NSUB>
struct __attribute__((aligned(16))) FwdSmem {
  char k[KBUF][SUBN * NSUB * D * 2];
  char v[VBUF][SUBN * NSUB * D * 2];
};

// NW wavefronts (4 or 8) of 32 query rows each; key tiles of NSUB 32-key
// subtiles (2: 64 keys, two workgroups per CU; 1: 32 keys, whose smaller
// register set and LDS footprint let three workgroups share a CU).  With
// NSUB = 1 the second subtile's statements below are compiled out.
template <int D, bool CAUSAL, int NW = 4, bool PACK = false, int NSUB = 2>
__device__ __forceinline__ void fa2_fwd_bf16(const bf16* __restrict__ q, const bf16* __restrict__ k,
                             const bf16* __restrict__ v, bf16* __restrict__ o,
                             float* __restrict__ lse, int nq, int nk, float scale, int hq, int hkv,
                             int num_m_blocks, int total_blocks, int o_merged,
                             const float2* __restrict__ rope_cs) {
  constexpr int BN = SUBN * NSUB;      // keys per tile
  constexpr int BM = 32 * NW;          // query rows per workgroup
  constexpr int NT = 64 * NW;          // threads
  constexpr int DC = D / 16;           // d-chunks of 16 for QK^T
  constexpr int DT = D / 32;           // d-tiles of 32 for PV
  constexpr int CPR = D / 8;           // 16-byte chunks per row
  constexpr int TCH = BN * CPR / NT;   // chunks per thread per tile (K and V each)
  constexpr int LSTEP = NT * 16;       // bytes of one load across the workgroup
  constexpr int TILE = BN * D * 2;     // bytes per tile
  __shared__ FwdSmem<D, NSUB> sm;

  const int tid = threadIdx.x;
  // wave-uniform (an SGPR): every branch on it is a scalar branch
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;

  const int id = xcd_remap(blockIdx.x, total_blocks);
  int bh, rank;
  // causal blocks: heads in groups of 4 (measured 1.02-1.06x at B16 Hq32 Hkv8
  // S512 and B4 S2048 against pairs; equal blocks gain nothing from it)
  pair_order<CAUSAL ? 4 : 2>(id, num_m_blocks, total_blocks / num_m_blocks, bh, rank);
  const int mb = num_m_blocks - 1 - rank;  // the last query block is the heaviest
  // bhq: this wavefront's (b, q head); wrow0: its first query row; blk_end:
  // one past the workgroup's last row.  GQA-packed (PACK, NW = hq / hkv): bh
  // is a (b, kv head), every wavefront takes the same 32 rows of its own q
  // head of the group; otherwise bh is a (b, q head) and wavefront w takes
  // rows 32 w of the block's BM.
  int bhq, wrow0, blk_end;
  long kvh;
  if constexpr (PACK) {
    const int b = bh / hkv;
    kvh = bh;
    bhq = b * hq + (bh - b * hkv) * NW + wave;
    wrow0 = mb * 32;
    blk_end = wrow0 + 32;
  } else {
    const int b = bh / hq, h = bh - b * hq;
    kvh = (long)b * hkv + h / (hq / hkv);
    bhq = bh;
    wrow0 = mb * BM + wave * 32;
    blk_end = mb * BM + BM;
  }
  const int qrow = wrow0 + l32;
  const int wave_qmax = wrow0 + 31;

  const bf16* kb = k + kvh * (long)nk * D;
  const bf16* vb = v + kvh * (long)nk * D;

  // ---- Q rows -> registers (B operand) -------------------------------------
  // rows past nq load row nq - 1: computed, never stored.  rope_cs: q is the
  // fused QKV projection [B, nq, (hq + 2 hkv) D], whose q heads are rotated
  // here (row r at position r, its (cos, sin) from the table) as the split
  // kernel would rotate them, and rounded to bf16 as it would store them
  bf16x8 qreg[DC];
  // rope_cs: the (cos, sin) of the lane's pairs (columns 16 c + 8 g .. + 7
  // are pairs 8 c + 4 g .. + 3: two float4 per c, pairs 8 c + 4 g + 2 m,
  // +1 in qcs[2 c + m]), applied once the first tiles are requested, so
  // that their loads do not wait for Q's
  float4 qcs[2 * DC];
  {
    const int qr = min(qrow, nq - 1);
    const bf16* qp;
    if (rope_cs) {
      const int qb = bhq / hq, qh = bhq - qb * hq;
      qp = q + ((long)qb * nq + qr) * ((hq + 2 * hkv) * D) + qh * D + 8 * g;
    } else {
      qp = q + ((long)bhq * nq + qr) * D + 8 * g;
    }
#pragma unroll
    for (int c = 0; c < DC; ++c) qreg[c] = as_bf16x8(*reinterpret_cast<const u32x4*>(qp + 16 * c));
    if (rope_cs) {
      // the table's row blocks of 32 positions: load i of the lane (row qr,
      // half g) is float4 ((qr / 32) * 2 DC + i) * 64 + (qr % 32) * 2 + g,
      // one KiB per load instruction of the wavefront
      const float4* cs = reinterpret_cast<const float4*>(rope_cs) +
                         (long)(qr >> 5) * (2 * DC * 64) + (qr & 31) * 2 + g;
#pragma unroll
      for (int i = 0; i < 2 * DC; ++i) qcs[i] = cs[64 * i];
    }
  }
  auto rotate_q = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      const u32x4 w = __builtin_bit_cast(u32x4, qreg[c]);
      u32x4 r;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 t = qcs[2 * c + j / 2];  // (cos, sin) of pairs 2 (j / 2), +1
        const float cn = j % 2 ? t.z : t.x, sn = j % 2 ? t.w : t.y;
        float o0, o1;
        rope_rotate(bf16lo(w[j]), bf16hi(w[j]), cn, sn, o0, o1);
        r[j] = pack_bf16x2(o0, o1);
      }
      qreg[c] = as_bf16x8(r);
    }
  };

  int kend = nk;
  if (CAUSAL) kend = min(nk, blk_end);
  const int n_iter = (kend + BN - 1) / BN;
  // causal: the workgroup's tiles past this wavefront's last row are fully
  // masked for it; it computes only the first n_live (wave-uniform)
  const int n_live = CAUSAL ? min(n_iter, wave_qmax / BN + 1) : n_iter;

  // ---- direct global -> LDS tile loads --------------------------------------
  // buffer_load ... lds (MUBUF, not FLAT: LDS waits elsewhere in the loop keep
  // partial counts), address = SGPR descriptor of the head + SGPR tile offset
  // + one VGPR per lane.  Load i of a wave writes LDS chunks
  // (i*NT + wave*64 + lane) of the tile; each lane fetches the tile chunk
  // that the swizzle puts there.  Adding 256 chunks (16 lines) leaves both
  // swizzles unchanged, so a lane's chunks are one byte offset plus i * LSTEP.
  const uint32_t k_src = swz<SWZ_ROW, D>(wave * 64 + lane) * 16;
  const uint32_t v_src = swz<SWZ_DUAL, D>(wave * 64 + lane) * 16;
  const auto krsrc = make_rsrc(kb, nk * D * 2);
  const auto vrsrc = make_rsrc(vb, nk * D * 2);
  // it: tile index; koff / voff: byte offsets of its K and V buffers.  Rows
  // past the sequence lie outside the descriptors' ranges and load as zeros:
  // their scores are masked, and P = 0 times V = 0 adds nothing.
  auto load_tile = [&](int it, int koff, int voff) {
    char* kdst = sm.k[0] + koff + wave * 64 * 16;
    char* vdst = sm.v[0] + voff + wave * 64 * 16;
    const int sbase = it * BN * D * 2;
#pragma unroll
    for (int i = 0; i < TCH; ++i) {
      dma16(krsrc, kdst + i * LSTEP, k_src, sbase + i * LSTEP);
      dma16(vrsrc, vdst + i * LSTEP, v_src, sbase + i * LSTEP);
    }
  };

  // ---- LDS read offsets (bytes within a tile) -------------------------------
  // K: lane reads row 32*kt + l32, column chunk 2c + g.
  int k_off[DC];
#pragma unroll
  for (int c = 0; c < DC; ++c) {
    k_off[c] = swz<SWZ_ROW, D>(l32 * CPR + 2 * c + g) * 16;
    // opaque to the optimiser: known-zero high bits would turn buffer base +
    // offset into an OR, which is not folded into the read's immediate offset
    pin(k_off[c]);
  }
  // V^T: lane p of 16-lane group G reads row 4g + p/4 (+8, +16hh, +32kt) and
  // 8 bytes at column 32t + 16(G%2) + 4(p%4); rows differing by 8 share the
  // swizzle, so only the column tile t needs its own offset.
  const int vr = 4 * g + ((lane & 15) >> 2);
  int v_off[DT][2];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int row = 8 * e + 4 * g + ((lane & 15) >> 2);
      const int col = 32 * t + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
      v_off[t][e] = swz<SWZ_DUAL, D>(row * CPR + col / 8) * 16 + (col % 8) * 2;
      pin(v_off[t][e]);
    }
  constexpr int ROW8 = 8 * D * 2;  // bytes of 8 rows (a swizzle-invariant step)

  // ---- running state ---------------------------------------------------------
  f32x16 acc_o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc_o[t] = f32x16{};
  // m_run: the exponent offset of P, the row maximum of the first tile,
  // raised only by a tile whose P would reach 2^31 (then O and l rescale)
  float m_run = -INFINITY;
  // this lane's partial row sums (its 16 of every 32 keys), two chains
  float l_run = 0.0f, l_run2 = 0.0f;
  const float sl2 = scale * kLog2e;

  // P of the previous tile: the B operand of its delayed PV product
  uint32_t pprev[NSUB][8];
  uint32_t pnew[NSUB][8];

  // PV product j = (kt, hh, t): A = V^T rows t of keys 32kt + 16hh .. +16,
  // two transpose reads; B = P of those keys
  constexpr int NJ = 2 * NSUB * DT;
  constexpr int VPF = 2;  // V fragments are read this many products ahead
  auto pv_read = [&](const char* vt, int j) {
    const int t = j % DT, hh = (j / DT) & 1, kt = j / (2 * DT);
    const char* p = vt + (4 * kt + 2 * hh) * ROW8;
    u32x2 a0 = lds_read_tr(p + v_off[t][0]), a1 = lds_read_tr(p + v_off[t][1]);
    return u32x4{a0[0], a0[1], a1[0], a1[1]};
  };
  auto pv_mfma = [&](int j, u32x4 a) {
    const int t = j % DT, hh = (j / DT) & 1, kt = j / (2 * DT);
    bf16x8 bop = as_bf16x8(u32x4{pprev[kt][4 * hh], pprev[kt][4 * hh + 1],
                                 pprev[kt][4 * hh + 2], pprev[kt][4 * hh + 3]});
    acc_o[t] = mfma32(as_bf16x8(a), bop, acc_o[t]);
  };

  // S^T = K Q^T for the NSUB 32-key subtiles of a tile (interleaved
  // chains, K fragments read KPF steps ahead)
  auto qk = [&](const char* kt0, f32x16& s0, f32x16& s1) {
    constexpr int KPF = 2;
    s0 = f32x16{};
    if constexpr (NSUB == 2) s1 = f32x16{};
    u32x4 ra[DC], rb[DC];
#pragma unroll
    for (int c = 0; c < KPF; ++c) {
      ra[c] = *reinterpret_cast<const u32x4*>(kt0 + k_off[c]);
      if constexpr (NSUB == 2) rb[c] = *reinterpret_cast<const u32x4*>(kt0 + 32 * D * 2 + k_off[c]);
    }
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      if (c + KPF < DC) {
        ra[c + KPF] = *reinterpret_cast<const u32x4*>(kt0 + k_off[c + KPF]);
        if constexpr (NSUB == 2)
          rb[c + KPF] = *reinterpret_cast<const u32x4*>(kt0 + 32 * D * 2 + k_off[c + KPF]);
      }
      s0 = mfma32(as_bf16x8(ra[c]), qreg[c], s0);
      if constexpr (NSUB == 2) s1 = mfma32(as_bf16x8(rb[c]), qreg[c], s1);
    }
    sched_group(kDsRead, NSUB * KPF);
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      if (c + KPF < DC) sched_group(kDsRead, NSUB);
      sched_group(kMfma, NSUB);
    }
  };

  // raw scores of keys past the sequence or (causal) past the row -> -inf;
  // only tiles that reach past nk or past the wave's first row need it
  auto mask = [&](int kbase, f32x16& s0, f32x16& s1) {
    if ((kbase + BN > nk) || (CAUSAL && kbase + BN - 1 > wrow0)) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        int key = kbase + 8 * (r >> 2) + 4 * g + (r & 3);
        if (key >= nk || (CAUSAL && key > qrow)) s0[r] = -INFINITY;
        if constexpr (NSUB == 2) {
          key += 32;
          if (key >= nk || (CAUSAL && key > qrow)) s1[r] = -INFINITY;
        }
      }
    }
  };

  // Row max of a tile in four pieces, the last one followed by the online-
  // softmax update (first tile, or a tile redone): m_run raised to the
  // tile's maximum where that is larger, alpha the factor of O and l (O is
  // scaled before the next product: grow), m_use the exponent offset of P.
  float mxa, mxb, alpha = 1.0f, m_use = 0.0f;
  bool grow = false;
  auto max_piece = [&](int u, const f32x16& s0, const f32x16& s1) {
    if (u == 0) {
      mxa = max3(s0[0], s0[1], s0[2]);
      if constexpr (NSUB == 2) mxb = max3(s1[0], s1[1], s1[2]);
    }
#pragma unroll
    for (int r = (u == 0 ? 3 : 4 * u + 1); r < 4 * u + 5 && r < 15; r += 2) {
      mxa = max3(mxa, s0[r], s0[r + 1]);
      if constexpr (NSUB == 2) mxb = max3(mxb, s1[r], s1[r + 1]);
    }
    if (u == 3) {
      float mx;
      if constexpr (NSUB == 2) mx = max3(mxa, mxb, max3(s0[15], s1[15], s1[15]));
      else mx = fmaxf(mxa, s0[15]);
      mx = max3(mx, other_half(mx), mx);
      const float m_tile = mx * sl2;  // scale > 0, so max(scale*s) = scale*max(s)
      const float m_new = fmaxf(m_run, m_tile);
      // 0 on a row's first tile; exactly 1 where the maximum is unchanged
      alpha = m_new == -INFINITY ? 1.0f : fast_exp2(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
      l_run2 *= alpha;
      m_use = m_run == -INFINITY ? 0.0f : m_run;
      grow = true;
    }
  };
  // softmax of element pair q, the bf16 P that the PV product consumes
  // added into one of two row-sum chains.  NSUB = 2: pairs 0..15, half q%2
  // (s0 / s1), rows 2(q/2), +1 (la: s0's keys, lb: s1's); NSUB = 1: pairs
  // 0..7, elements 2q, 2q+1 of s0 (la: even pairs, lb: odd)
  auto sm_pair = [&](const f32x16& s0, const f32x16& s1, int q, float& la, float& lb) {
    if constexpr (NSUB == 2) {
      const int hf = q & 1, r = (q >> 1) * 2;
      const float x0 = hf ? s1[r] : s0[r], x1 = hf ? s1[r + 1] : s0[r + 1];
      const uint32_t w = pack_bf16x2(fast_exp2(__builtin_fmaf(x0, sl2, -m_use)),
                                     fast_exp2(__builtin_fmaf(x1, sl2, -m_use)));
      pnew[hf][r >> 1] = w;
      if (hf) lb = add_bf16x2(w, lb);
      else la = add_bf16x2(w, la);
    } else {
      const uint32_t w = pack_bf16x2(fast_exp2(__builtin_fmaf(s0[2 * q], sl2, -m_use)),
                                     fast_exp2(__builtin_fmaf(s0[2 * q + 1], sl2, -m_use)));
      pnew[0][q] = w;
      if (q & 1) lb = add_bf16x2(w, lb);
      else la = add_bf16x2(w, la);
    }
  };
  // the tile's partial row sums are checked before they join l: a tile with
  // a sum at or above 2^31 (or not finite) is redone with its maximum
  auto check_tile = [&](const f32x16& s0, const f32x16& s1, float& la, float& lb) {
    if (__any(!(fmaxf(la, lb) < kPmax))) {  // wave-uniform and rare
#pragma unroll
      for (int u = 0; u < 4; ++u) max_piece(u, s0, s1);
      la = 0.0f;
      lb = 0.0f;
#pragma unroll
      for (int q = 0; q < 8 * NSUB; ++q) sm_pair(s0, s1, q, la, lb);
    }
    l_run += la;
    l_run2 += lb;
  };
  // the product after which softmax pair q is issued (8 NSUB pairs over NJ
  // products)
  auto pair_slot = [](int q) { return q * NJ / (8 * NSUB); };
  auto rescale_o = [&]() {
#pragma unroll
    for (int t = 0; t < DT; ++t) acc_o[t] *= alpha;
  };


  // ---- first tile: scores and P only ----
  if (n_iter > 0) {
    // tile 1 is requested with tile 0, before the first wait: its latency
    // overlaps the first tile's, and the first tile's products wait only for
    // the Q rows and tile 0 (tile 1's 2 TCH loads, issued last, may still fly)
    load_tile(0, 0, 0);
    if (n_iter > 1) {
      load_tile(1, TILE, TILE);
      __builtin_amdgcn_s_waitcnt(kVmWaitLgkm0<2 * TCH>());
    } else {
      __builtin_amdgcn_s_waitcnt(0);
    }
    // (the barrier alone: __syncthreads would wait for tile 1's loads too)
    barrier_only();
    if (rope_cs) rotate_q();
    f32x16 s0, s1;
    qk(sm.k[0], s0, s1);
    mask(0, s0, s1);
#pragma unroll
    for (int u = 0; u < 4; ++u) max_piece(u, s0, s1);
    grow = false;  // O is still zero: no scaling due
#pragma unroll
    for (int q = 0; q < 8 * NSUB; ++q) sm_pair(s0, s1, q, l_run, l_run2);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pprev[0][i] = pnew[0][i];
      if constexpr (NSUB == 2) pprev[1][i] = pnew[1][i];
    }
    __builtin_amdgcn_s_waitcnt(0);  // this thread's loads of tile 1 have landed
    __syncthreads();
  }

  // ---- steady state: QK of tile it; then the PV product of tile it-1 on the
  //      matrix cores interleaved with tile it's softmax on the VALU ----
  // Tile it's K sits in buffer it % 2, its V in buffer it % 3.  The loop is
  // unrolled over the 6 tiles after which both rotations repeat, so every LDS
  // address is a lane offset plus a constant (the read's immediate offset)
  // instead of one address add per read.
  auto tile_step = [&](int it, auto KB, auto VP) {
    constexpr int kb = decltype(KB)::value;  // K buffer of tile it
    constexpr int vp = decltype(VP)::value;  // V buffer of tile it - 1
    const int kbase = it * BN;
    f32x16 s0, s1;
    qk(sm.k[kb], s0, s1);
    mask(kbase, s0, s1);
    // a maximum raised by tile it-1 scales O before tile it-1's product
    if (grow) {
      rescale_o();
      grow = false;
    }
    float la = 0.0f, lb = 0.0f;

    // issue order, fenced: V reads VPF products ahead; each product followed
    // by its share of the exponentials.
    // Tile it+1's loads go out halfway through the PV products: issued
    // before the score products they held up the first MFMAs; issued right
    // after them, a quarter or three quarters of the way through the PV
    // products, the kernel took 1.6, 1.4 and 2.8 % more cycles (measured).
    const char* vt = sm.v[vp];
    u32x4 va[NJ];
#pragma unroll
    for (int j = 0; j < VPF; ++j) va[j] = pv_read(vt, j);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (j + VPF < NJ) va[j + VPF] = pv_read(vt, j + VPF);
      pv_mfma(j, va[j]);
#pragma unroll
      for (int q = 0; q < 8 * NSUB; ++q)
        if (pair_slot(q) == j) sm_pair(s0, s1, q, la, lb);
      if (j == NJ / 2 && it + 1 < n_iter)
        load_tile(it + 1, ((kb + 1) % KBUF) * TILE, ((vp + 2) % VBUF) * TILE);
      __builtin_amdgcn_sched_barrier(0);
    }
    check_tile(s0, s1, la, lb);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pin(pnew[0][i]);
      if constexpr (NSUB == 2) pin(pnew[1][i]);
      pprev[0][i] = pnew[0][i];
      if constexpr (NSUB == 2) pprev[1][i] = pnew[1][i];
    }
    pin(l_run);
    pin(l_run2);
    __builtin_amdgcn_s_waitcnt(0);  // this thread's loads of tile it+1 have landed
    __syncthreads();
  };
  {
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    int it = 1;
    for (; it + 6 <= n_live; it += 6) {
      tile_step(it, I1{}, I0{});
      tile_step(it + 1, I0{}, I1{});
      tile_step(it + 2, I1{}, I2{});
      tile_step(it + 3, I0{}, I0{});
      tile_step(it + 4, I1{}, I1{});
      tile_step(it + 5, I0{}, I2{});
    }
    // the last (n_live - 1) % 6 tiles (same buffer sequence)
    if (it < n_live) tile_step(it, I1{}, I0{});
    if (it + 1 < n_live) tile_step(it + 1, I0{}, I1{});
    if (it + 2 < n_live) tile_step(it + 2, I1{}, I2{});
    if (it + 3 < n_live) tile_step(it + 3, I0{}, I0{});
    if (it + 4 < n_live) tile_step(it + 4, I1{}, I1{});
  }
  if (n_iter > 0) {
    if (grow) rescale_o();
    const char* vt = sm.v[0] + ((n_live - 1) % VBUF) * TILE;  // tile n_live-1's V
#pragma unroll
    for (int j = 0; j < NJ; ++j) pv_mfma(j, pv_read(vt, j));
    // a wavefront whose rows end before the workgroup's last tiles still
    // loads its share of them and meets the workgroup at each of their
    // barriers (tile t + 1 goes to K buffer (t + 1) % 2, V buffer (t + 1) % 3,
    // as in the steps)
    for (int t = n_live; t < n_iter; ++t) {
      if (t + 1 < n_iter) load_tile(t + 1, ((t + 1) % KBUF) * TILE, ((t + 1) % VBUF) * TILE);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
  }

  // ---- epilogue ----
  l_run += l_run2;
  const float l_tot = l_run + other_half(l_run);
  const float inv = 1.0f / l_tot;  // rows past nq: never stored
  // O goes through LDS (the K/V buffers, free once every wavefront's last PV
  // product has read its tile): each wavefront writes its 32 x D tile, the
  // 16-byte chunk c of row r at chunk c ^ (r % CPR) of that row, and reads it
  // back a whole row per CPR lanes, so one store writes 64 / CPR complete
  // rows instead of 32 scattered 16-byte pieces (stored straight from the
  // accumulators, the O rows kept each workgroup ~2 us longer on its CU)
  static_assert(sizeof(FwdSmem<D, NSUB>) >= NW * 32 * D * 2, "O tiles fit the K/V buffers");
  constexpr int RPI = 64 / CPR;  // rows per store
  __builtin_amdgcn_s_waitcnt(kVmWaitLgkm0<63>());  // this wavefront's LDS reads
  barrier_only();
  char* ot = reinterpret_cast<char*>(&sm) + wave * (32 * D * 2);
  // byte offsets, formed here (the empty asm keeps them out of the loop,
  // where they would be live across it): the write of chunk c is
  // wa ^ (c << 4) (row l32, half g), the read of store kk is
  // (ra ^ ((kk % (CPR / RPI)) * RPI << 4)) + kk * RPI * 2 D (row kk RPI +
  // lane / CPR, chunk lane % CPR), both XORs on bits 4.. of a row's chunk
  // index only
  const int ln = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const int lr = ln & 31;
  int wa = lr * (2 * D) + 8 * (ln >> 5) + ((lr & (CPR - 1)) << 4);
  int ra = (ln / CPR) * (2 * D) + (((ln % CPR) ^ (ln / CPR)) << 4);
  // O's layout: [B, Hq, Sq, D] (rows of a head D apart), or, o_merged,
  // [B, Sq, Hq, D], the merged-heads layout (rows Hq D apart)
  const int rs = o_merged ? hq * D : D;
  int sa = (ln / CPR) * rs + 8 * (ln % CPR);  // element offset of the lane's store
  asm volatile("" : "+v"(wa), "+v"(ra), "+v"(sa));
#pragma unroll
  for (int t = 0; t < DT; ++t) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // this lane's d = 32 t + 8 j + 4 g .. + 3: half g of chunk 4 t + j
      const u32x2 w = {pack_bf16x2(acc_o[t][4 * j] * inv, acc_o[t][4 * j + 1] * inv),
                       pack_bf16x2(acc_o[t][4 * j + 2] * inv, acc_o[t][4 * j + 3] * inv)};
      *reinterpret_cast<u32x2*>(ot + (wa ^ ((4 * t + j) << 4))) = w;
    }
  }
  const int hd = bhq % hq;  // this wavefront's q head within its batch row
  bf16* ob = o + (long)(bhq - hd) * nq * D + (long)wrow0 * rs + (long)hd * (o_merged ? D : nq * D);
#pragma unroll
  for (int kk = 0; kk < 32 / RPI; ++kk) {
    const u32x4 val = *reinterpret_cast<const u32x4*>(
        ot + (ra ^ (((kk % (CPR / RPI)) * RPI) << 4)) + kk * RPI * 2 * D);
    if (wrow0 + kk * RPI + ln / CPR < nq)
      *reinterpret_cast<u32x4*>(ob + kk * RPI * rs + sa) = val;
  }
  if (qrow < nq && g == 0) lse[(long)bhq * nq + qrow] = (m_run + __log2f(l_tot)) * kLn2;
}

}  // namespace

// One instance: name suffix, head dim, causal, wavefronts, GQA-packed, 32-key
// subtiles per tile, wavefronts per SIMD the register budget is sized for.
// At D = 128 the causal forms take 32-key tiles at three wavefronts per SIMD
// (168 VGPRs, 40 KiB LDS, three workgroups per CU): 2-7 % faster than 64-key
// tiles at two, which cover each other's MFMA and VALU phases less well;
// the bidirectional form keeps 64-key tiles (at 168 VGPRs it spills and ran
// 3 % slower).  At D = 64 the 64-key tiles already fit three wavefronts per
// SIMD (149-165 VGPRs): 5-6 % faster than at two, with the same output bits.
#define TEENY_FA2_FWD_BF16_K(SFX, D, C, NW, PACK, NSUB, WPE)                                   \
  extern "C" __global__ __launch_bounds__(64 * NW)                                               \
      __attribute__((amdgpu_waves_per_eu(WPE, WPE))) void teeny_fa2_fwd_bf16_d##D##_##SFX(       \
          const bf16* q, const bf16* k, const bf16* v, bf16* o, float* l, int nq, int nk,        \
          float scale, int hq, int hkv, int nmb, int total, int o_merged,                       \
          const float2* rope_cs) {                                                               \
    fa2_fwd_bf16<D, C, NW, PACK, NSUB>(q, k, v, o, l, nq, nk, scale, hq, hkv, nmb, total,        \
                                       o_merged, rope_cs);                                       \
  }

// 4 wavefronts, 128 query rows of one (b, q head) per workgroup
TEENY_FA2_FWD_BF16_K(c, 64, true, 4, false, 2, 3)
TEENY_FA2_FWD_BF16_K(n, 64, false, 4, false, 2, 3)
TEENY_FA2_FWD_BF16_K(c, 128, true, 4, false, 1, 3)
TEENY_FA2_FWD_BF16_K(n, 128, false, 4, false, 2, 2)

// 8 wavefronts, 256 query rows per workgroup (long GQA sequences)
TEENY_FA2_FWD_BF16_K(c_w8, 128, true, 8, false, 2, 2)
TEENY_FA2_FWD_BF16_K(n_w8, 128, false, 8, false, 2, 2)

// GQA-packed: one workgroup per (b, kv head, 32 query rows), wavefront w on
// q head kv head * NW + w (hq = NW hkv); every wavefront of a causal block
// ends on the same row, so none waits out the block's last tiles
TEENY_FA2_FWD_BF16_K(c_g4, 64, true, 4, true, 2, 3)
TEENY_FA2_FWD_BF16_K(c_g4, 128, true, 4, true, 1, 3)
TEENY_FA2_FWD_BF16_K(c_g8, 128, true, 8, true, 2, 2)

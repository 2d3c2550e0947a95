// bf16 flash-attention 2 forward on CDNA4 matrix cores (gfx950).
//
// Reference semantics: flash_attn2_causal_fwd (src/kernels/flash_attn2.rs:61-126)
// and the bidirectional forward (:57-58): O = softmax(scale * Q K^T [+ causal
// mask k > q]) V per query row, LSE = m + ln(l) in the natural-log,
// scaled-score domain (:121-122).  The reference is fp32 with one CTA per
// query row; this kernel keeps bf16 operands with fp32 accumulation and a
// fp32 online softmax.
//
// Tiling (one workgroup = 4 wavefronts = 128 query rows of one (b, h)):
//   * each wave owns 32 query rows; its Q rows live in registers as the
//     B operand of v_mfma_f32_32x32x16_bf16;
//   * K/V advance in tiles of 64 keys, double-buffered in LDS, both stored
//     row-major [key][d]; K is read as an A operand with 16-byte reads, V^T
//     with the LDS transpose read ds_read_b64_tr_b16 (see vt_operand);
//   * S^T = K Q^T puts one query row in each lane (lane % 32) and 16 keys per
//     lane per 32-key subtile, so the row max / row sum are in-lane plus one
//     exchange between the two lane halves;
//   * the fp32 accumulator of S^T, rounded to bf16, is already in the
//     B-operand layout of O^T += V^T P^T (keys are a summation index, so the
//     key order inside each 16-key chunk only has to agree between A and B);
//   * causal: key tiles past the block's last query row are skipped, subtiles
//     past a wave's last row are skipped, only diagonal tiles are masked;
//   * GQA: q head h reads kv head h / (Hq / Hkv);
//   * scheduling: block ids are remapped so one XCD works through whole heads
//     (K/V stay in that XCD's L2), heaviest causal blocks first.
// exp is exp2 with log2(e) folded into the scale (v_exp_f32).
#include "common.h"

namespace {

constexpr int BM = 128;  // query rows per workgroup
constexpr int BN = 64;   // keys per iteration
constexpr int KBUF = 2;  // K tiles in flight: read by QK(i), loading i+1
constexpr int VBUF = 3;  // V tiles: read by PV(i-1), waiting (i), loading (i+1)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kRescale = 8.0f;  // lazy-rescale threshold, log2 units

DEVI float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
DEVI bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }
DEVI f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

// ds_read_b64_tr_b16: within each 16-lane group, output lane i receives
// element (i % 4) of the 8-byte chunks addressed by lanes i/4, i/4+4, i/4+8
// and i/4+12 (measured on gfx950): lanes addressing a 4-row x 16-column block
// of a row-major tile receive it transposed, one column per lane.
DEVI u32x2 lds_read_tr(const char* p) {
  s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(p));
  return __builtin_bit_cast(u32x2, r);
}

// Tiles are stored unpadded, 16-byte chunk L = row * (D/8) + column-chunk,
// and XOR-swizzled within each 256-byte line (64 banks x 4 bytes):
//   K (read by rows, 16 bytes per lane):   position ^= line % 16
//   V (read by the 4-row transpose reads): position ^= 2 * (line % 4)
// so 16 lanes of either read touch distinct bank groups, and both swizzles
// repeat every 8 rows for D = 64 and D = 128 (the reads step by 8 rows).
template <bool VLAYOUT>
DEVI int swz_chunk(int L) {
  const int line = L >> 4, pos = L & 15;
  const int x = VLAYOUT ? ((line & 3) << 1) : (line & 15);
  return (line << 4) | (pos ^ x);
}

template <int D>
struct __attribute__((aligned(16))) FwdSmem {
  char k[KBUF][BN * D * 2];
  char v[VBUF][BN * D * 2];
};

template <int D, bool CAUSAL>
__device__ void fa2_fwd_bf16(const bf16* __restrict__ q, const bf16* __restrict__ k,
                             const bf16* __restrict__ v, bf16* __restrict__ o,
                             float* __restrict__ lse, int nq, int nk, float scale, int hq, int hkv,
                             int num_m_blocks, int total_blocks) {
  constexpr int DC = D / 16;           // d-chunks of 16 for QK^T
  constexpr int DT = D / 32;           // d-tiles of 32 for PV
  constexpr int CPR = D / 8;           // 16-byte chunks per row
  constexpr int TCH = BN * CPR / 256;  // chunks per thread per tile (K and V each)
  constexpr int TILE = BN * D * 2;     // bytes per tile
  __shared__ FwdSmem<D> sm;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;

  const int id = xcd_remap(blockIdx.x, total_blocks);
  const int bh = id / num_m_blocks;
  const int mb = num_m_blocks - 1 - (id - bh * num_m_blocks);
  const int b = bh / hq, h = bh - b * hq;
  const long kvh = (long)b * hkv + h / (hq / hkv);
  const int m0 = mb * BM;
  const int qrow = m0 + wave * 32 + l32;
  const int wave_qmax = m0 + wave * 32 + 31;

  const bf16* kb = k + kvh * (long)nk * D;
  const bf16* vb = v + kvh * (long)nk * D;

  // ---- Q rows -> registers (B operand) -------------------------------------
  bf16x8 qreg[DC];
  {
    const bool ok = qrow < nq;
    const bf16* qp = q + ((long)bh * nq + (ok ? qrow : 0)) * D + 8 * g;
#pragma unroll
    for (int c = 0; c < DC; ++c)
      qreg[c] = as_bf16x8(ok ? *reinterpret_cast<const u32x4*>(qp + 16 * c) : u32x4{0, 0, 0, 0});
  }

  int kend = nk;
  if (CAUSAL) kend = min(nk, m0 + BM);
  const int n_iter = (kend + BN - 1) / BN;

  // ---- direct global -> LDS tile loads --------------------------------------
  // Load i of a wave writes LDS chunks (i*256 + wave*64 + lane) of the tile;
  // each lane fetches the tile chunk that the swizzle puts there.
  int k_src[TCH], v_src[TCH];  // element offsets of those chunks within a tile
#pragma unroll
  for (int i = 0; i < TCH; ++i) {
    const int P = i * 256 + wave * 64 + lane;
    const int Lk = swz_chunk<false>(P), Lv = swz_chunk<true>(P);  // (an involution)
    k_src[i] = (Lk / CPR) * D + (Lk % CPR) * 8;
    v_src[i] = (Lv / CPR) * D + (Lv % CPR) * 8;
  }
  auto load_tile = [&](int it) {
    const int kbase = it * BN;
    char* kdst = sm.k[it % KBUF] + wave * 64 * 16;
    char* vdst = sm.v[it % VBUF] + wave * 64 * 16;
    const bf16* kt = kb + (long)kbase * D;
    const bf16* vt = vb + (long)kbase * D;
    const bool full = kbase + BN <= nk;
#pragma unroll
    for (int i = 0; i < TCH; ++i) {
      int ko = k_src[i], vo = v_src[i];
      if (!full) {  // rows past the sequence re-read its last row (masked later)
        ko = min(ko / D, nk - 1 - kbase) * D + ko % D;
        vo = min(vo / D, nk - 1 - kbase) * D + vo % D;
      }
      __builtin_amdgcn_global_load_lds((const void*)(kt + ko), (lds_void*)(kdst + i * 4096), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(vt + vo), (lds_void*)(vdst + i * 4096), 16, 0, 0);
    }
  };

  // ---- LDS read offsets (bytes within a tile) -------------------------------
  // K: lane reads row 32*kt + l32, column chunk 2c + g.
  int k_off[DC];
#pragma unroll
  for (int c = 0; c < DC; ++c) k_off[c] = swz_chunk<false>(l32 * CPR + 2 * c + g) * 16;
  // V^T: lane p of 16-lane group G reads row 4g + p/4 (+8, +16hh, +32kt) and
  // 8 bytes at column 32t + 16(G%2) + 4(p%4); rows differing by 8 share the
  // swizzle, so only the column tile t needs its own offset.
  const int vr = 4 * g + ((lane & 15) >> 2);
  int v_off[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    const int col = 32 * t + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    v_off[t] = swz_chunk<true>(vr * CPR + col / 8) * 16 + (col % 8) * 2;
  }
  constexpr int ROW8 = 8 * D * 2;  // bytes of 8 rows (a swizzle-invariant step)

  // ---- running state ---------------------------------------------------------
  f32x16 acc_o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc_o[t] = f32x16{};
  // m_run is raised lazily: only when some row of the wave sees a max more
  // than kRescale above it are O and l rescaled, so p = 2^(t - m_run) stays
  // below 2^kRescale (exact in fp32 and representable in bf16).
  float m_run = -INFINITY;
  float l_run = 0.0f;  // this lane's partial row sum (its 16 of every 32 keys)
  const float sl2 = scale * kLog2e;

  // P of the previous tile (B operand of its delayed PV) and its activity
  uint32_t pprev[2][8];
  bool prev_act0 = false, prev_act1 = false;
  int prev_buf = 0;

  auto pv = [&](int vbuf, bool a1) {
    const char* vt = sm.v[vbuf];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      if (kt == 1 && !a1) break;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        bf16x8 bop = as_bf16x8(u32x4{pprev[kt][4 * hh], pprev[kt][4 * hh + 1],
                                     pprev[kt][4 * hh + 2], pprev[kt][4 * hh + 3]});
#pragma unroll
        for (int t = 0; t < DT; ++t) {
          const char* p = vt + v_off[t] + (4 * kt + 2 * hh) * ROW8;
          u32x2 a0 = lds_read_tr(p);
          u32x2 a1v = lds_read_tr(p + ROW8);
          acc_o[t] = mfma32(as_bf16x8(u32x4{a0[0], a0[1], a1v[0], a1v[1]}), bop, acc_o[t]);
        }
      }
    }
  };

  if (n_iter > 0) load_tile(0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  for (int it = 0; it < n_iter; ++it) {
    const int kbase = it * BN;
    if (it + 1 < n_iter) load_tile(it + 1);
    // causal: a tile whose first key is past this wave's last row is all masked
    const bool act0 = !(CAUSAL && kbase > wave_qmax);
    const bool act1 = act0 && kbase + 32 < nk && !(CAUSAL && kbase + 32 > wave_qmax);

    f32x16 s0 = f32x16{}, s1 = f32x16{};
    if (act0) {
      // ---- S^T = K Q^T for the two 32-key subtiles (chains interleaved) ----
      const char* kt0 = sm.k[it % KBUF];
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        u32x4 a0 = *reinterpret_cast<const u32x4*>(kt0 + k_off[c]);
        s0 = mfma32(as_bf16x8(a0), qreg[c], s0);
        if (act1) {
          u32x4 a1 = *reinterpret_cast<const u32x4*>(kt0 + 32 * D * 2 + k_off[c]);
          s1 = mfma32(as_bf16x8(a1), qreg[c], s1);
        }
      }
    }
    // ---- the previous tile's O^T += V^T P^T runs while this tile's softmax
    //      occupies the VALU ----
    if (prev_act0) pv(prev_buf, prev_act1);

    if (act0) {
      // ---- masking (boundary tiles only): raw scores -> -inf ----
      const bool need_mask = (kbase + BN > nk) || (CAUSAL && kbase + BN - 1 > m0 + wave * 32);
      if (need_mask) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          int key = kbase + 8 * (r >> 2) + 4 * g + (r & 3);
          if (key >= nk || (CAUSAL && key > qrow)) s0[r] = -INFINITY;
          key += 32;
          if (!act1 || key >= nk || (CAUSAL && key > qrow)) s1[r] = -INFINITY;
        }
      } else if (!act1) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s1[r] = -INFINITY;
      }
      // ---- online softmax, log2 domain, lazy rescale ----
      float mx = fmaxf(s0[0], s1[0]);
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmaxf(mx, fmaxf(s0[r], s1[r]));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_tile = mx * sl2;  // scale > 0, so max(scale*s) = scale*max(s)
      const bool grow = m_tile > m_run + kRescale;
      if (__any(grow)) {
        const float m_new = fmaxf(m_run, m_tile);
        // 0 on a row's first tile; 1 for rows that did not grow (or saw no key)
        const float alpha = m_new == -INFINITY ? 1.0f : fast_exp2(m_run - m_new);
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int t = 0; t < DT; ++t) acc_o[t] *= alpha;
      }
      const float m_use = m_run == -INFINITY ? 0.0f : m_run;
      float psum = 0.0f;
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        float p0 = fast_exp2(__builtin_fmaf(s0[r], sl2, -m_use));
        float p1 = fast_exp2(__builtin_fmaf(s0[r + 1], sl2, -m_use));
        float p2 = fast_exp2(__builtin_fmaf(s1[r], sl2, -m_use));
        float p3 = fast_exp2(__builtin_fmaf(s1[r + 1], sl2, -m_use));
        psum += (p0 + p1) + (p2 + p3);
        pprev[0][r >> 1] = pack_bf16x2(p0, p1);
        pprev[1][r >> 1] = pack_bf16x2(p2, p3);
      }
      l_run += psum;
    }
    prev_act0 = act0;
    prev_act1 = act1;
    prev_buf = it % VBUF;

    __builtin_amdgcn_s_waitcnt(0);  // this thread's loads of tile it+1 have landed
    __syncthreads();
  }
  if (prev_act0) pv(prev_buf, prev_act1);

  // ---- epilogue ----
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  if (qrow < nq) {
    const float inv = 1.0f / l_tot;
    bf16* orow = o + ((long)bh * nq + qrow) * D;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        int d = 32 * t + 8 * j + 4 * g;
        u32x2 w = {pack_bf16x2(acc_o[t][4 * j] * inv, acc_o[t][4 * j + 1] * inv),
                   pack_bf16x2(acc_o[t][4 * j + 2] * inv, acc_o[t][4 * j + 3] * inv)};
        *reinterpret_cast<u32x2*>(orow + d) = w;
      }
    }
    if (g == 0) lse[(long)bh * nq + qrow] = (m_run + __log2f(l_tot)) * kLn2;
  }
}

}  // namespace

#define TEENY_FA2_FWD_BF16_INST(D)                                                               \
  extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))      \
  void teeny_fa2_fwd_bf16_d##D##_c(                                                              \
      const bf16* q, const bf16* k, const bf16* v, bf16* o, float* l, int nq, int nk,            \
      float scale, int hq, int hkv, int nmb, int total) {                                        \
    fa2_fwd_bf16<D, true>(q, k, v, o, l, nq, nk, scale, hq, hkv, nmb, total);                    \
  }                                                                                              \
  extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))      \
  void teeny_fa2_fwd_bf16_d##D##_n(                                                              \
      const bf16* q, const bf16* k, const bf16* v, bf16* o, float* l, int nq, int nk,            \
      float scale, int hq, int hkv, int nmb, int total) {                                        \
    fa2_fwd_bf16<D, false>(q, k, v, o, l, nq, nk, scale, hq, hkv, nmb, total);                   \
  }

TEENY_FA2_FWD_BF16_INST(64)
TEENY_FA2_FWD_BF16_INST(128)

// bf16 decode attention on the matrix cores (gfx950): one new query row per
// (b, q head) against the first n_keys rows of the KV cache, split over the
// keys (flash-decoding); the partials (max, sum, unnormalised O) are merged
// by teeny_decode_attn_combine (llama.hip).
//
// One wavefront per (key split, b, kv head).  The q heads of the GQA group
// (Hq / Hkv <= 32 of them) are the rows of the forward kernel's layout: their
// Q rows are the B operand of v_mfma_f32_32x32x16_bf16 in registers (rows
// past the group are zero), 32-key tiles of K and V stream into LDS by
// buffer_load ... lds two tiles deep, S^T = K Q^T puts one head in each lane,
// and O^T += V^T P^T reads V^T with the LDS transpose read.  Most of the 32
// MFMA rows are padding; at 8 MFMAs per 8 KiB of K the matrix cores still
// outrun HBM several times, and the kernel is bound by reading the cache.
// Reference: the reference recomputes the whole prefix every step
// (examples/llama_generate.rs:373-381); this is the last row of that
// attention (flash_attn2.rs:61-126) evaluated once.
#include "cdna4.h"

namespace {

constexpr int TK = 32;  // keys per tile
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// s_waitcnt immediate for vmcnt(0) alone (expcnt and lgkmcnt fields at their
// maximum: not waited for), and for lgkmcnt(0) alone
constexpr int kVmcnt0 = (7 << 4) | (15 << 8);
constexpr int kLgkmcnt0 = 15 | (3 << 14) | (7 << 4);

template <int D>
struct __attribute__((aligned(16))) DecSmem {
  char k[2][TK * D * 2];
  char v[2][TK * D * 2];
};

// n_keys = the n_keys argument, or min(*n_past + 1, n_keys) when n_past is
// given (n_keys is then the grid's max_keys), clamped to the cache.
template <int D>
__device__ void decode_mfma(const bf16* __restrict__ q, const bf16* __restrict__ kc,
                            const bf16* __restrict__ vc, float* __restrict__ pm,
                            float* __restrict__ pl, float* __restrict__ po, int hq, int hkv,
                            const int* __restrict__ n_past, int n_keys, int cache_len,
                            int keys_per_split, float scale) {
  constexpr int DC = D / 16, DT = D / 32, CPR = D / 8;
  constexpr int TILE = TK * D * 2;   // bytes of a K or V tile
  constexpr int NLD = TILE / 1024;   // 16-byte-per-lane loads per tile
  __shared__ DecSmem<D> sm;

  const int lane = threadIdx.x, l32 = lane & 31, g = lane >> 5;
  const int split = blockIdx.x, n_split = gridDim.x;
  const int kvh = blockIdx.y, b = kvh / hkv, hk = kvh - b * hkv;
  const int group = hq / hkv;
  if (n_past) n_keys = min(min(*n_past + 1, n_keys), cache_len);
  n_keys = __builtin_amdgcn_readfirstlane(n_keys);  // wave-uniform
  const int k0 = split * keys_per_split;
  const int k1 = min(k0 + keys_per_split, n_keys);
  const long qrow0 = (long)b * hq + (long)hk * group;  // first q head of the group

  bf16x8 qreg[DC];
#pragma unroll
  for (int c = 0; c < DC; ++c)
    qreg[c] = l32 < group ? as_bf16x8(*reinterpret_cast<const u32x4*>(
                                q + (qrow0 + l32) * D + 16 * c + 8 * g))
                          : as_bf16x8(u32x4{0, 0, 0, 0});

  const auto krs = make_rsrc(kc + (long)kvh * cache_len * D, cache_len * D * 2);
  const auto vrs = make_rsrc(vc + (long)kvh * cache_len * D, cache_len * D * 2);
  // load i writes LDS chunk i*64 + lane of a tile, which holds tile chunk swz(.)
  uint32_t ksrc[NLD], vsrc[NLD];
#pragma unroll
  for (int i = 0; i < NLD; ++i) {
    ksrc[i] = swz<SWZ_ROW, D>(i * 64 + lane) * 16;
    vsrc[i] = swz<SWZ_DUAL, D>(i * 64 + lane) * 16;
  }
  // keys t0 .. t0+TK-1; rows at or past n_keys re-read row n_keys - 1: they
  // are masked (P = 0), and a row never written (or stale, or NaN) past
  // n_keys must not reach the P V product, where 0 * NaN would be NaN
  auto load = [&](int t0, int buf) {
    // uniform; said explicitly, or the compiler wraps each load in a
    // per-lane loop over the values of a vector register
    const int soff = __builtin_amdgcn_readfirstlane(t0 * D * 2);
    if (t0 + TK <= n_keys) {
#pragma unroll
      for (int i = 0; i < NLD; ++i) {
        dma16(krs, sm.k[buf] + i * 1024, ksrc[i], soff);
        dma16(vrs, sm.v[buf] + i * 1024, vsrc[i], soff);
      }
    } else {
      const int lastrow = n_keys - 1 - t0;
#pragma unroll
      for (int i = 0; i < NLD; ++i) {
        dma16(krs, sm.k[buf] + i * 1024,
              min((int)ksrc[i] / (2 * D), lastrow) * (2 * D) + ksrc[i] % (2 * D), soff);
        dma16(vrs, sm.v[buf] + i * 1024,
              min((int)vsrc[i] / (2 * D), lastrow) * (2 * D) + vsrc[i] % (2 * D), soff);
      }
    }
  };

  int k_off[DC];
#pragma unroll
  for (int c = 0; c < DC; ++c) k_off[c] = swz<SWZ_ROW, D>(l32 * CPR + 2 * c + g) * 16;
  int v_off[DT][2];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int row = 8 * e + 4 * g + ((lane & 15) >> 2);
      const int col = 32 * t + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
      v_off[t][e] = swz<SWZ_DUAL, D>(row * CPR + col / 8) * 16 + (col % 8) * 2;
    }

  f32x16 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f32x16{};
  float m = -INFINITY, l = 0.0f;  // log2-domain max of scale * score; this lane's sum
  const float sl2 = scale * kLog2e;
  const int n_tiles = k0 < k1 ? (k1 - k0 + TK - 1) / TK : 0;
  if (n_tiles > 0) load(k0, 0);
  for (int it = 0; it < n_tiles; ++it) {
    const int buf = it & 1, t0 = k0 + it * TK;
    // tile it has landed; tile it + 1 streams in while it is used.  (Waiting
    // for a partial count here instead made the compiler add a wait for
    // every LDS load in flight before the first LDS read.)
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    if (it + 1 < n_tiles) load(t0 + TK, buf ^ 1);
    const char* kt = sm.k[buf];
    const char* vt = sm.v[buf];
    // all K reads first (one LDS latency per tile, not one per product)
    u32x4 kr[DC];
#pragma unroll
    for (int c = 0; c < DC; ++c) kr[c] = *reinterpret_cast<const u32x4*>(kt + k_off[c]);
    f32x16 s = f32x16{};
#pragma unroll
    for (int c = 0; c < DC; ++c) s = mfma32(as_bf16x8(kr[c]), qreg[c], s);
    sched_group(kDsRead, DC);
    sched_group(kMfma, DC);
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (t0 + 8 * (r >> 2) + 4 * g + (r & 3) >= k1) s[r] = -INFINITY;
    float mx = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
    mx = fmaxf(mx, other_half(mx));
    const float m_new = fmaxf(m, mx * sl2);  // finite: tile it has a key below k1
    const float alpha = fast_exp2(m - m_new);
    m = m_new;
    l *= alpha;
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] *= alpha;
    uint32_t pb[8];
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      pb[r >> 1] = pack_bf16x2(fast_exp2(__builtin_fmaf(s[r], sl2, -m)),
                               fast_exp2(__builtin_fmaf(s[r + 1], sl2, -m)));
      l = add_bf16x2(pb[r >> 1], l);
    }
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const bf16x8 bop = as_bf16x8(u32x4{pb[4 * hh], pb[4 * hh + 1], pb[4 * hh + 2], pb[4 * hh + 3]});
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const char* p = vt + hh * 16 * D * 2;
        u32x2 a0 = lds_read_tr(p + v_off[t][0]), a1 = lds_read_tr(p + v_off[t][1]);
        acc[t] = mfma32(as_bf16x8(u32x4{a0[0], a0[1], a1[0], a1[1]}), bop, acc[t]);
      }
    }
  }
  const float l_tot = l + other_half(l);
  if (l32 < group) {
    const long row = (qrow0 + l32) * n_split + split;
    if (g == 0) {
      pm[row] = n_tiles > 0 ? m * kLn2 : -INFINITY;  // natural-log units for the merge
      pl[row] = l_tot;
    }
    float* orow = po + row * D;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) orow[32 * t + 8 * (r >> 2) + 4 * g + (r & 3)] = acc[t][r];
  }
}

// The whole attention of a graph-captured decode step in one launch, one
// workgroup of 8 wavefronts per (b, kv head):
//   1. the group's q heads and the kv head's k, v rows are summed from the
//      QKV projection's K-split slabs (in slab order, rounded to bf16 as the
//      unsplit product is stored), RoPE is applied at position n_past to q
//      and k (qkv_rope_split's arithmetic); q, k and v stay in LDS;
//   2. the cache rows 0 .. min(n_past + 1, cache_len) - 1 are split between
//      the 8 wavefronts, each running decode_mfma's loop on its own LDS
//      buffer of one 32-key tile.  Every wavefront's first tile is requested
//      before step 1, so the two latencies overlap; the cache is read only
//      below row n_past (rows at or past it load as zeros: outside the
//      descriptors' ranges) and the wavefront whose tile holds row n_past
//      copies the new k, v row from LDS into it;
//   3. the 8 partials (max, sum, unnormalised O) are merged in LDS and
//      o [B, Hq, D] is stored, and the new k, v row is written to the cache
//      (row n_past, when it is below cache_len) for the next steps.
// It replaces the QKV split, the split-K decode kernel and the combine
// kernel of the unfused path with one launch and no partials in HBM.
constexpr int kDqWaves = 8;

template <int D>
struct __attribute__((aligned(16))) DecQkvSmem {
  union {
    struct {
      char k[kDqWaves][TK * D * 2];
      char v[kDqWaves][TK * D * 2];
    } t;
    struct {
      float m[kDqWaves][32];
      float l[kDqWaves][32];
      float o[kDqWaves][32 * D];
    } c;
  } u;
  bf16 q[32 * D];      // the group's RoPE'd q rows
  bf16 kv[2][D];       // the new cache row: k (RoPE'd), v
  float cs[D / 2][2];  // (cos, sin) of the pair angles at the new position
};

template <int D>
__device__ void decode_qkv_attn(const float* __restrict__ parts, int n_parts, long part_stride,
                                bf16* __restrict__ kc, bf16* __restrict__ vc,
                                bf16* __restrict__ o, int hq, int hkv,
                                const int* __restrict__ n_past, int cache_len, float ln_base,
                                float scale) {
  constexpr int DC = D / 16, DT = D / 32, CPR = D / 8;
  constexpr int TILE = TK * D * 2;  // bytes of a K or V tile
  constexpr int NLD = TILE / 1024;  // 16-byte-per-lane loads per tile
  constexpr int VN = 8;             // bf16 per 16-byte vector
  __shared__ DecQkvSmem<D> sm;

  const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, g = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kvh = blockIdx.x, b = kvh / hkv, hk = kvh - b * hkv;
  const int group = hq / hkv;
  const int htot = hq + 2 * hkv;
  const int pos = __builtin_amdgcn_readfirstlane(*n_past);
  const int n_keys = __builtin_amdgcn_readfirstlane(min(pos + 1, cache_len));

  // this wavefront's keys k0 .. k1 - 1, in 32-key tiles through its LDS buffer
  const int kpw = ((n_keys + kDqWaves - 1) / kDqWaves + TK - 1) / TK * TK;
  const int k0 = wave * kpw;
  const int k1 = min(k0 + kpw, n_keys);
  const int n_tiles = k0 < k1 ? (k1 - k0 + TK - 1) / TK : 0;
  // the cache up to row pos - 1 (the rows this step reads from it); rows at
  // or past pos lie outside the ranges and load as zeros
  const int rows_old = max(0, min(pos, cache_len));
  const auto krs = make_rsrc(kc + (long)kvh * cache_len * D, rows_old * D * 2);
  const auto vrs = make_rsrc(vc + (long)kvh * cache_len * D, rows_old * D * 2);
  uint32_t ksrc[NLD], vsrc[NLD];
#pragma unroll
  for (int i = 0; i < NLD; ++i) {
    ksrc[i] = swz<SWZ_ROW, D>(i * 64 + lane) * 16;
    vsrc[i] = swz<SWZ_DUAL, D>(i * 64 + lane) * 16;
  }
  // K or V rows t0 .. t0+TK-1 into this wavefront's buffer (keys at or past
  // n_keys are masked)
  auto load_k = [&](int t0) {
    const int soff = __builtin_amdgcn_readfirstlane(t0 * D * 2);
#pragma unroll
    for (int i = 0; i < NLD; ++i) dma16(krs, sm.u.t.k[wave] + i * 1024, ksrc[i], soff);
  };
  auto load_v = [&](int t0) {
    const int soff = __builtin_amdgcn_readfirstlane(t0 * D * 2);
#pragma unroll
    for (int i = 0; i < NLD; ++i) dma16(vrs, sm.u.t.v[wave] + i * 1024, vsrc[i], soff);
  };
  if (n_tiles > 0) {
    load_k(k0);
    load_v(k0);
  }

  // ---- 1. q, k, v of position pos -------------------------------------------
  // A thread sums the K-split slabs of up to two 16-byte items (group + 2
  // rows of D / VN items; group <= 32).  The (cos, sin) of the D / 2 pair
  // angles at position pos are the same for every q head and k: the last
  // D / 2 threads evaluate them once, into LDS, while the slab loads fly
  // (evaluated per item they were 4 serial exp / sincos chains per thread).
  constexpr int NT = kDqWaves * 64;
  const int n_items = (group + 2) * (D / VN);
  float in[2][VN];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int i = tid + r * NT;
    if (i < n_items) {
      const int hh = i / (D / VN), vv = i - hh * (D / VN);
      const int row = hh < group ? hk * group + hh : (hh == group ? hq + hk : hq + hkv + hk);
      ld_parts<bf16, VN>(parts + ((long)b * htot + row) * D + vv * VN, part_stride, n_parts,
                         in[r]);
    }
  }
  if (tid >= NT - D / 2) {
    const int kk = tid - (NT - D / 2);
    float sn, cn;
    rope_cos_sin(pos, kk, rope_c(ln_base, D), cn, sn);
    sm.cs[kk][0] = cn;
    sm.cs[kk][1] = sn;
  }
  // the table is in LDS; the barrier alone (no wait for the tile loads in
  // flight)
  __builtin_amdgcn_s_waitcnt(kLgkmcnt0);
  barrier_only();
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int i = tid + r * NT;
    if (i < n_items) {
      const int hh = i / (D / VN), vv = i - hh * (D / VN);
      float out[VN];
      if (hh <= group) {  // q and k: RoPE on the interleaved pairs
#pragma unroll
        for (int j = 0; j < VN / 2; ++j) {
          const int kk = vv * (VN / 2) + j;
          const float cn = sm.cs[kk][0], sn = sm.cs[kk][1];
          rope_rotate(in[r][2 * j], in[r][2 * j + 1], cn, sn, out[2 * j], out[2 * j + 1]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < VN; ++j) out[j] = in[r][j];
      }
      if (hh < group) Vec16<bf16>::store(sm.q + hh * D + vv * VN, out);
      else Vec16<bf16>::store(sm.kv[hh - group] + vv * VN, out);
    }
  }
  // q and the new k, v row are in LDS; the barrier alone (no wait for the
  // tile loads in flight)
  __builtin_amdgcn_s_waitcnt(kLgkmcnt0);
  barrier_only();

  bf16x8 qreg[DC];
#pragma unroll
  for (int cc = 0; cc < DC; ++cc)
    qreg[cc] = l32 < group ? as_bf16x8(*reinterpret_cast<const u32x4*>(
                                 sm.q + l32 * D + 16 * cc + 8 * g))
                           : as_bf16x8(u32x4{0, 0, 0, 0});

  // ---- 2. attention over this wavefront's keys (decode_mfma's loop) ---------
  int k_off[DC];
#pragma unroll
  for (int cc = 0; cc < DC; ++cc) k_off[cc] = swz<SWZ_ROW, D>(l32 * CPR + 2 * cc + g) * 16;
  int v_off[DT][2];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int r = 8 * e + 4 * g + ((lane & 15) >> 2);
      const int col = 32 * t + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
      v_off[t][e] = swz<SWZ_DUAL, D>(r * CPR + col / 8) * 16 + (col % 8) * 2;
    }

  f32x16 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f32x16{};
  float m = -INFINITY, l = 0.0f;  // log2-domain max of scale * score; this lane's sum
  const float sl2 = scale * kLog2e;
  const char* kt = sm.u.t.k[wave];
  const char* vt = sm.u.t.v[wave];
  // Tile it's K arrives before its V: the K of tile it + 1 is requested as
  // soon as tile it's K fragments are in registers, its V after tile it's V
  // reads, so the next tile's scores and softmax run while its V is still
  // in flight (in order: K(it), V(it), then K(it + 1), V(it + 1)).
  for (int it = 0; it < n_tiles; ++it) {
    const int t0 = k0 + it * TK;
    const bool has_pos = t0 <= pos && pos < t0 + TK;
    // the tile holding row pos gets the new k (then v) row from LDS (tile
    // chunk r * CPR + c sits at LDS chunk swz(r * CPR + c)); the reads below
    // are issued after these writes by the same wavefront
    __builtin_amdgcn_s_waitcnt(kVmWait<NLD>());  // K of tile it has landed
    if (has_pos && lane < CPR) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(sm.kv[0] + 8 * lane);
      *reinterpret_cast<u32x4*>((char*)kt + swz<SWZ_ROW, D>((pos - t0) * CPR + lane) * 16) = w;
    }
    u32x4 kr[DC];
#pragma unroll
    for (int cc = 0; cc < DC; ++cc) kr[cc] = *reinterpret_cast<const u32x4*>(kt + k_off[cc]);
    f32x16 s = f32x16{};
#pragma unroll
    for (int cc = 0; cc < DC; ++cc) s = mfma32(as_bf16x8(kr[cc]), qreg[cc], s);
    sched_group(kDsRead, DC);
    sched_group(kMfma, DC);
    // every K read has returned: the next tile's K may refill the buffer
    __builtin_amdgcn_s_waitcnt(kLgkmcnt0);
    if (it + 1 < n_tiles) load_k(t0 + TK);
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (t0 + 8 * (r >> 2) + 4 * g + (r & 3) >= k1) s[r] = -INFINITY;
    float mx = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
    mx = fmaxf(mx, other_half(mx));
    const float m_new = fmaxf(m, mx * sl2);  // finite: tile it has a key below k1
    const float alpha = fast_exp2(m - m_new);
    m = m_new;
    l *= alpha;
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] *= alpha;
    uint32_t pb[8];
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      pb[r >> 1] = pack_bf16x2(fast_exp2(__builtin_fmaf(s[r], sl2, -m)),
                               fast_exp2(__builtin_fmaf(s[r + 1], sl2, -m)));
      l = add_bf16x2(pb[r >> 1], l);
    }
    // V of tile it has landed (K of tile it + 1 may still fly)
    if (it + 1 < n_tiles) __builtin_amdgcn_s_waitcnt(kVmWait<NLD>());
    else __builtin_amdgcn_s_waitcnt(kVmcnt0);
    if (has_pos && lane < CPR) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(sm.kv[1] + 8 * lane);
      *reinterpret_cast<u32x4*>((char*)vt + swz<SWZ_DUAL, D>((pos - t0) * CPR + lane) * 16) = w;
    }
    u32x4 va[2][DT];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const char* pp = vt + hh * 16 * D * 2;
        u32x2 a0 = lds_read_tr(pp + v_off[t][0]), a1 = lds_read_tr(pp + v_off[t][1]);
        va[hh][t] = u32x4{a0[0], a0[1], a1[0], a1[1]};
      }
    // every V read has returned: the next tile's V may refill the buffer
    // while the products run
    __builtin_amdgcn_s_waitcnt(kLgkmcnt0);
    if (it + 1 < n_tiles) load_v(t0 + TK);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const bf16x8 bop = as_bf16x8(u32x4{pb[4 * hh], pb[4 * hh + 1], pb[4 * hh + 2], pb[4 * hh + 3]});
#pragma unroll
      for (int t = 0; t < DT; ++t) acc[t] = mfma32(as_bf16x8(va[hh][t]), bop, acc[t]);
    }
  }
  const float l_tot = l + other_half(l);

  // ---- 3. merge the wavefronts' partials ------------------------------------
  __syncthreads();  // every wavefront is done with its tiles
  if (l32 < group) {
    if (g == 0) {
      sm.u.c.m[wave][l32] = m;  // -inf for a wavefront without keys
      sm.u.c.l[wave][l32] = l_tot;
    }
    float* orow = sm.u.c.o[wave] + l32 * D;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) orow[32 * t + 8 * (r >> 2) + 4 * g + (r & 3)] = acc[t][r];
  }
  __syncthreads();
  for (int i = tid; i < group * D; i += kDqWaves * 64) {
    const int hh = i / D, d = i - hh * D;
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDqWaves; ++w) mm = fmaxf(mm, sm.u.c.m[w][hh]);
    float num = 0.0f, den = 0.0f;
#pragma unroll
    for (int w = 0; w < kDqWaves; ++w) {
      const float e = fast_exp2(sm.u.c.m[w][hh] - mm);  // 0 for a wavefront without keys
      num += e * sm.u.c.o[w][hh * D + d];
      den += e * sm.u.c.l[w][hh];
    }
    o[((long)b * hq + hk * group + hh) * D + d] = (bf16)(num / den);
  }
  // the new k, v row to the cache, for the next steps
  if (pos >= 0 && pos < cache_len && tid < 2 * CPR) {
    const int c = tid % CPR;
    bf16* cache = tid < CPR ? kc : vc;
    *reinterpret_cast<u32x4*>(cache + ((long)kvh * cache_len + pos) * D + 8 * c) =
        *reinterpret_cast<const u32x4*>(sm.kv[tid >= CPR] + 8 * c);
  }
}

}  // namespace

#define TEENY_DECODE_BF16_INST(D)                                                                \
  extern "C" __global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2)))          \
  void teeny_decode_mfma_bf16_d##D(                                                             \
      const bf16* q, const bf16* kc, const bf16* vc, float* pm, float* pl, float* po, int hq,    \
      int hkv, const int* n_past, int n_keys, int cache_len, int keys_per_split, float scale) {  \
    decode_mfma<D>(q, kc, vc, pm, pl, po, hq, hkv, n_past, n_keys, cache_len, keys_per_split,   \
                   scale);                                                                       \
  }

TEENY_DECODE_BF16_INST(64)
TEENY_DECODE_BF16_INST(128)

#define TEENY_DECODE_QKV_INST(D)                                                                 \
  extern "C" __global__ __launch_bounds__(512) void teeny_decode_qkv_attn_bf16_d##D(            \
      const float* parts, int n_parts, long part_stride, bf16* kc, bf16* vc, bf16* o, int hq,    \
      int hkv, const int* n_past, int cache_len, float ln_base, float scale) {                   \
    decode_qkv_attn<D>(parts, n_parts, part_stride, kc, vc, o, hq, hkv, n_past, cache_len,      \
                       ln_base, scale);                                                          \
  }

TEENY_DECODE_QKV_INST(64)
TEENY_DECODE_QKV_INST(128)

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
// maximum: not waited for)
constexpr int kVmcnt0 = (7 << 4) | (15 << 8);

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

// Llama attention plumbing around the flash-attention kernels.
//
// teeny_qkv_rope_split: the fused QKV projection output [B, S, (Hq+2Hkv)*D]
//   -> Q [B, Hq, S, D] with RoPE, and K (RoPE) / V appended to a KV cache
//   [B, Hkv, cache_len, D] at positions pos0 .. pos0+S-1.  One pass over HBM
//   replaces the reference's three TransposeHeadsOp and two RopeOp launches
//   (src/layers/attention.rs:97-123; transpose_heads.rs:49-71, rope.rs:57-97)
//   with the same arithmetic: interleaved pairs, theta = fp32(pos) *
//   fp32(exp_f64(fp32(k) * (-2 ln_base / D))), position = absolute position.
//   pos0 may instead be read from device memory (a captured decode step whose
//   position advances between replays); rows whose position falls outside
//   the cache are then not written to it.  With q_out null only the cache
//   rows are written (the bf16 prompt attention then reads Q from qkv and
//   rotates it as it loads it, with teeny_rope_table's (cos, sin)).
//
// teeny_decode_attn_*: one new query row per (b, q head) against the first
//   n_keys cached keys (flash-decoding: split-K partials over 256-key chunks,
//   then a log-sum-exp merge).  The reference has no KV cache and recomputes
//   the whole prefix every step (examples/llama_generate.rs:373-381); this is
//   the same attention row evaluated once.
#include "common.h"

namespace {

constexpr int kThreads = 256;
// The slab form (decode steps, whose QKV comes as K-split slabs): a
// workgroup covers 4 head rows (of Hq + 2 Hkv) x 4 positions with a (cos,
// sin) table in LDS, so that many workgroups share the slab reads.

// PARTS: qkv is the sum of n_parts fp32 slabs part_stride apart (the QKV
// projection split over K), rounded to T as the unsplit product is stored.
template <typename T, bool PARTS = false, int kRows = 16, int kPos = 16>
__device__ void qkv_rope_split(const T* __restrict__ qkv, T* __restrict__ q_out,
                               T* __restrict__ k_cache, T* __restrict__ v_cache, int seq,
                               const int* __restrict__ pos_dev, int pos0, int cache_len, int hq,
                               int hkv, int head_dim, float ln_base,
                               const float* __restrict__ parts = nullptr, int n_parts = 0,
                               long part_stride = 0) {
  extern __shared__ float2 cs_tab[];  // [kPos][head_dim / 2]
  const int half = head_dim / 2;
  const int s0 = blockIdx.x * kPos;
  const int htot = hq + 2 * hkv;
  const int rows_per_b = (htot + kRows - 1) / kRows;
  const int b = blockIdx.y / rows_per_b;
  const int h0 = (blockIdx.y - b * rows_per_b) * kRows;
  constexpr int VN = Vec16<T>::N;
  const int vpr = head_dim / VN;
  const int total = kRows * kPos * vpr;
  auto source = [&](int i, int& v, int& p, int& hh, int& s) {  // false: nothing to do
    v = i % vpr;
    const int r = i / vpr;
    p = r % kPos;
    hh = h0 + r / kPos;
    s = s0 + p;
    return s < seq && hh < htot;
  };
  auto load = [&](int v, int hh, int s, float* in) {
    const long src = ((long)b * seq + s) * htot * head_dim + (long)hh * head_dim + v * VN;
    if constexpr (PARTS)
      ld_parts<T, VN>(parts + src, part_stride, n_parts, in);
    else
      Vec16<T>::load(qkv + src, in);
  };
  // this thread's first item is read before the rotation table is built, so
  // the two latencies overlap (a decode step has one item per thread)
  int v, p, hh, s;
  float in[VN];
  const bool first = (int)threadIdx.x < total && source(threadIdx.x, v, p, hh, s);
  if (first) load(v, hh, s, in);

  if (pos_dev) pos0 += *pos_dev;
  const float c = rope_c(ln_base, head_dim);
  for (int i = threadIdx.x; i < kPos * half; i += kThreads) {
    int pp = i / half, k = i - pp * half;
    if (s0 + pp >= seq) break;  // i grows with pp: no later entry is needed either
    float sn, cn;
    rope_cos_sin(pos0 + s0 + pp, k, c, cn, sn);
    cs_tab[i] = make_float2(cn, sn);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < total; i += kThreads) {
    if (i != (int)threadIdx.x) {
      if (!source(i, v, p, hh, s)) continue;
      load(v, hh, s, in);
    } else if (!first) {
      continue;
    }
    if (hh >= hq && (pos0 + s < 0 || pos0 + s >= cache_len)) continue;  // outside the cache
    T* dst;
    if (hh < hq)
      dst = q_out + (((long)b * hq + hh) * seq + s) * head_dim;
    else if (hh < hq + hkv)
      dst = k_cache + (((long)b * hkv + (hh - hq)) * cache_len + pos0 + s) * head_dim;
    else
      dst = v_cache + (((long)b * hkv + (hh - hq - hkv)) * cache_len + pos0 + s) * head_dim;
    float out[VN];
    if (hh < hq + hkv) {
      const float2* cs = cs_tab + p * half + v * (VN / 2);
#pragma unroll
      for (int j = 0; j < VN / 2; ++j) {
        rope_rotate(in[2 * j], in[2 * j + 1], cs[j].x, cs[j].y, out[2 * j], out[2 * j + 1]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < VN; ++j) out[j] = in[j];
    }
    Vec16<T>::store(dst + v * VN, out);
  }
}

// The prompt form: a thread owns one 16-byte vector column (position s,
// pairs v*VN/2 ..) of kQkvHeads consecutive head rows of a qkv row.  It
// issues those loads first, evaluates its VN/2 (cos, sin) pairs while they
// are in flight, then rotates (q and k heads) or copies (v heads) and stores
// them: no LDS table, no barrier, the transcendental work amortised over the
// heads (the standalone RoPE kernel's layout).  Consecutive threads take
// consecutive vectors of a row, then consecutive positions, so every load
// and store is a run of whole rows.
constexpr int kQkvHeads = 8;

template <typename T>
__device__ void qkv_rope_rows(const T* __restrict__ qkv, T* __restrict__ q_out,
                              T* __restrict__ k_cache, T* __restrict__ v_cache, int seq,
                              const int* __restrict__ pos_dev, int pos0, int cache_len, int hq,
                              int hkv, int head_dim, float ln_base) {
  constexpr int VN = Vec16<T>::N;
  const int vpr = head_dim / VN;  // vectors per head row (the host keeps it <= kThreads)
  const int ppw = kThreads / vpr;
  const int v = threadIdx.x % vpr;
  const int s = blockIdx.x * ppw + threadIdx.x / vpr;
  const int htot = hq + 2 * hkv;
  // q_out null: the K and V rows only (the attention reads Q from qkv itself)
  const int hbase = q_out ? 0 : hq;
  const int groups = (htot - hbase + kQkvHeads - 1) / kQkvHeads;
  const int b = blockIdx.y / groups;
  const int h0 = hbase + (blockIdx.y - b * groups) * kQkvHeads;
  if (s >= seq || (int)threadIdx.x >= ppw * vpr) return;
  const T* src = qkv + (((long)b * seq + s) * htot + h0) * head_dim + v * VN;
  float in[kQkvHeads][VN];
#pragma unroll
  for (int h = 0; h < kQkvHeads; ++h)
    if (h0 + h < htot) Vec16<T>::load(src + (long)h * head_dim, in[h]);

  if (pos_dev) pos0 += *pos_dev;
  const int pos = pos0 + s;
  float cn[VN / 2], sn[VN / 2];
  if (h0 < hq + hkv) {  // some head of the group is rotated
    const float c = rope_c(ln_base, head_dim);
#pragma unroll
    for (int j = 0; j < VN / 2; ++j) rope_cos_sin(pos, v * (VN / 2) + j, c, cn[j], sn[j]);
  }
#pragma unroll
  for (int h = 0; h < kQkvHeads; ++h) {
    const int hh = h0 + h;
    if (hh >= htot) break;
    if (hh >= hq && (pos < 0 || pos >= cache_len)) continue;  // outside the cache
    T* dst;
    if (hh < hq)
      dst = q_out + (((long)b * hq + hh) * seq + s) * head_dim;
    else if (hh < hq + hkv)
      dst = k_cache + (((long)b * hkv + (hh - hq)) * cache_len + pos) * head_dim;
    else
      dst = v_cache + (((long)b * hkv + (hh - hq - hkv)) * cache_len + pos) * head_dim;
    float out[VN];
    if (hh < hq + hkv) {
#pragma unroll
      for (int j = 0; j < VN / 2; ++j) {
        rope_rotate(in[h][2 * j], in[h][2 * j + 1], cn[j], sn[j], out[2 * j], out[2 * j + 1]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < VN; ++j) out[j] = in[h][j];
    }
    Vec16<T>::store(dst + v * VN, out);
  }
}

// ---------------------------------------------------------------------------
// Decode attention
// ---------------------------------------------------------------------------
constexpr int kChunk = 256;  // keys per split-K workgroup
constexpr int kMaxGroup = 16;
constexpr int kMaxD = 128;

// grid (n_chunks, B * Hkv); q [B, Hq, D], caches [B, Hkv, cache_len, D].
// Partials: m, l [B*Hq, n_chunks]; o [B*Hq, n_chunks, D] (unnormalised).
// n_keys = the n_keys argument, or min(*n_past + 1, n_keys) (the cached keys
// plus the new one, at most the grid's max_keys) when n_past is given,
// clamped to the cache.
template <typename T>
__device__ void decode_partial(const T* __restrict__ q, const T* __restrict__ kc,
                               const T* __restrict__ vc, float* __restrict__ pm,
                               float* __restrict__ pl, float* __restrict__ po, int hq, int hkv,
                               const int* __restrict__ n_past, int n_keys, int cache_len,
                               int head_dim, float scale) {
  if (n_past) n_keys = min(min(*n_past + 1, n_keys), cache_len);
  __shared__ float qs[kMaxGroup][kMaxD];
  __shared__ float ps[kMaxGroup][kChunk];
  __shared__ float red[kMaxGroup][kThreads / 64];
  __shared__ float ohalf[kMaxGroup][kMaxD];
  const int group = hq / hkv;
  const int kvh = blockIdx.y;  // b * hkv + hk
  const int b = kvh / hkv, hk = kvh - b * hkv;
  const int chunk = blockIdx.x, n_chunks = gridDim.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const long qh0 = (long)b * hq + (long)hk * group;  // first q head of the group
  for (int i = tid; i < group * head_dim; i += kThreads)
    qs[i / head_dim][i % head_dim] = (float)q[(qh0 + i / head_dim) * head_dim + i % head_dim];
  __syncthreads();

  // scores: one key per thread
  const int key = chunk * kChunk + tid;
  const bool valid = key < n_keys;
  float sc[kMaxGroup];
#pragma unroll
  for (int g = 0; g < kMaxGroup; ++g) sc[g] = 0.0f;
  if (valid) {
    const T* krow = kc + ((long)kvh * cache_len + key) * head_dim;
    constexpr int VN = Vec16<T>::N;
    for (int d0 = 0; d0 < head_dim; d0 += VN) {
      float kv[VN];
      Vec16<T>::load(krow + d0, kv);
#pragma unroll
      for (int g = 0; g < kMaxGroup; ++g) {
        if (g >= group) break;
#pragma unroll
        for (int j = 0; j < VN; ++j) sc[g] += qs[g][d0 + j] * kv[j];
      }
    }
  }
  // per-head chunk max and sum
  float mloc[kMaxGroup];
#pragma unroll
  for (int g = 0; g < kMaxGroup; ++g) {
    if (g >= group) break;
    float s = valid ? sc[g] * scale : -INFINITY;
    sc[g] = s;
    float m = wave_max(s);
    if (lane == 0) red[g][wave] = m;
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < kMaxGroup; ++g) {
    if (g >= group) break;
    float m = red[g][0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) m = fmaxf(m, red[g][w]);
    mloc[g] = m;
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < kMaxGroup; ++g) {
    if (g >= group) break;
    float p = valid ? expf(sc[g] - mloc[g]) : 0.0f;
    ps[g][tid] = p;
    float l = wave_sum(p);
    if (lane == 0) red[g][wave] = l;
  }
  __syncthreads();
  // O[g][d] = sum_k p[g][k] V[k][d]: thread = (d, key half)
  const int d = tid % head_dim;
  const int part = tid / head_dim;             // which slice of the chunk's keys
  const int nparts = kThreads / head_dim;      // 2 for D=128, 4 for D=64
  const int kper = kChunk / nparts;
  float acc[kMaxGroup];
#pragma unroll
  for (int g = 0; g < kMaxGroup; ++g) acc[g] = 0.0f;
  if (part < nparts) {
    const int kbeg = chunk * kChunk + part * kper;
    const int kend = min(kbeg + kper, n_keys);
    for (int kk = kbeg; kk < kend; ++kk) {
      float vv = (float)vc[((long)kvh * cache_len + kk) * head_dim + d];
      const int j = kk - chunk * kChunk;
#pragma unroll
      for (int g = 0; g < kMaxGroup; ++g) {
        if (g >= group) break;
        acc[g] += ps[g][j] * vv;
      }
    }
  }
  // reduce the key slices through LDS (slices 1.. add into slice 0)
  for (int sl = 1; sl < nparts; ++sl) {
    if (part == sl) {
#pragma unroll
      for (int g = 0; g < kMaxGroup; ++g) {
        if (g >= group) break;
        ohalf[g][d] = acc[g];
      }
    }
    __syncthreads();
    if (part == 0) {
#pragma unroll
      for (int g = 0; g < kMaxGroup; ++g) {
        if (g >= group) break;
        acc[g] += ohalf[g][d];
      }
    }
    __syncthreads();
  }
  if (part == 0) {
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) {
      if (g >= group) break;
      const long row = (qh0 + g) * n_chunks + chunk;
      po[row * head_dim + d] = acc[g];
      if (d == 0) {
        float l = 0.0f;
#pragma unroll
        for (int w = 0; w < kThreads / 64; ++w) l += red[g][w];
        pm[row] = mloc[g];
        pl[row] = l;
      }
    }
  }
}

// grid B*Hq, block head_dim threads: merge the chunk partials.  The partials
// of kGroup chunks are loaded together (one memory wait per group) and folded
// into a running maximum: acc and l are scaled by e^(m_old - m_new) when a
// group raises it.
template <typename T>
__device__ void decode_combine(const float* __restrict__ pm, const float* __restrict__ pl,
                               const float* __restrict__ po, T* __restrict__ o, int n_chunks,
                               int head_dim) {
  constexpr int kGroup = 16;
  const long row = blockIdx.x;
  const int d = threadIdx.x;
  const float* rm = pm + row * n_chunks;
  const float* rl = pl + row * n_chunks;
  const float* ro = po + row * n_chunks * head_dim + d;
  float m = -INFINITY, l = 0.0f, acc = 0.0f;
  for (int c0 = 0; c0 < n_chunks; c0 += kGroup) {
    float mv[kGroup], lv[kGroup], ov[kGroup];
#pragma unroll
    for (int c = 0; c < kGroup; ++c) {  // chunks past the end re-read the last one
      const int cc = min(c0 + c, n_chunks - 1);
      mv[c] = rm[cc];
      lv[c] = rl[cc];
      ov[c] = ro[(long)cc * head_dim];
    }
    float gm = m;
#pragma unroll
    for (int c = 0; c < kGroup; ++c) gm = fmaxf(gm, mv[c]);
    if (gm == -INFINITY) continue;  // no keys yet
    const float r = expf(m - gm);   // 0 while m is -inf
    l *= r;
    acc *= r;
#pragma unroll
    for (int c = 0; c < kGroup; ++c)
      if (c0 + c < n_chunks) {
        const float w = expf(mv[c] - gm);
        l += lv[c] * w;
        acc += ov[c] * w;
      }
    m = gm;
  }
  o[row * head_dim + d] = (T)(acc / l);
}

// Row argmax: one workgroup of 1024 threads per row, 16-byte loads; the
// last index of the maximum, as the reference's greedy_sample
// (examples/llama_generate.rs:252-257, Iterator::max_by); NaN, on which the
// reference's comparison panics, counts as the maximum.
constexpr int kArgThreads = 1024;
template <typename T>
__device__ void argmax_rows(const T* __restrict__ x, long long* __restrict__ out, int cols) {
  __shared__ float bv[kArgThreads / 64];
  __shared__ int bi[kArgThreads / 64];
  const T* row = x + (long)blockIdx.x * cols;
  float v = -INFINITY;
  int idx = -1;
  // a beats b: larger, or NaN over a number, or equal with the larger index
  // (the reference's Iterator::max_by keeps the last of equal maxima)
  auto better = [](float a, int ia, float b, int ib) {
    const bool an = a != a, bn = b != b;
    if (an || bn) return an && (!bn || ia > ib);
    return a > b || (a == b && ia > ib);
  };
  constexpr int VN = Vec16<T>::N;
  if (cols % VN == 0 && (reinterpret_cast<uintptr_t>(row) & 15) == 0) {
    // U vectors (64 values) per thread requested before the first
    // comparison.  A thread meets its indices in increasing order, so
    // `x >= v` keeps the last of equal maxima (-0 and +0 compare equal, as
    // in the reference) and NaN, which compares false, is tracked apart;
    // branch-free, one compare and two selects per value (the comparison
    // through `better` made every value a divergent branch, ~20 µs a row)
    constexpr int U = 64 / VN, STEP = kArgThreads * VN;
    int nan_idx = -1;
    for (int c0 = threadIdx.x * VN; c0 < cols; c0 += U * STEP) {
      float a[U][VN];
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (c0 + u * STEP < cols) Vec16<T>::load(row + c0 + u * STEP, a[u]);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u * STEP;
        if (c < cols)
#pragma unroll
          for (int j = 0; j < VN; ++j) {
            const float x = a[u][j];
            const bool ge = x >= v;
            v = ge ? x : v;
            idx = ge ? c + j : idx;
            nan_idx = x != x ? c + j : nan_idx;
          }
      }
    }
    if (nan_idx >= 0) {  // NaN is the maximum: the thread's last NaN
      v = __builtin_nanf("");
      idx = nan_idx;
    }
  } else {
    for (int c = threadIdx.x; c < cols; c += kArgThreads) {
      const float a = (float)row[c];
      if (better(a, c, v, idx)) {
        v = a;
        idx = c;
      }
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(v, off, 64);
    const int oi = __shfl_xor(idx, off, 64);
    if (better(ov, oi, v, idx)) {
      v = ov;
      idx = oi;
    }
  }
  if ((threadIdx.x & 63) == 0) {
    bv[threadIdx.x >> 6] = v;
    bi[threadIdx.x >> 6] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kArgThreads / 64; ++w)
      if (better(bv[w], bi[w], v, idx)) {
        v = bv[w];
        idx = bi[w];
      }
    out[blockIdx.x] = idx;
  }
}

// The (cos, sin) of every pair at positions 0 .. n_pos - 1 (n_pos a multiple
// of 32), what the kernels above evaluate for a row at that position, laid
// out for the bf16 forward's Q load: a lane of row r (r % 32 = lane % 32)
// and half g (lane / 32) rotates pairs 8 c + 4 g + 2 m + e (e, m in 0..1, c
// < head_dim / 16), and its load i = 2 c + m is the 16 bytes
// (cos, sin, cos, sin) of pairs e = 0, 1 at float4 index
// ((r / 32) * (head_dim / 8) + i) * 64 + (r % 32) * 2 + g, so that one load
// instruction of a wavefront reads one contiguous KiB.
__device__ void rope_table(float2* __restrict__ cs, int n_pos, int head_dim, float ln_base) {
  const int half = head_dim / 2;
  const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (long)n_pos * half) return;
  const int p = (int)(t / half), k = (int)(t - (long)p * half);
  float cn, sn;
  rope_cos_sin(p, k, rope_c(ln_base, head_dim), cn, sn);
  const int c = k >> 3, g = (k >> 2) & 1, m = (k >> 1) & 1, e = k & 1;
  const long f4 = ((long)(p >> 5) * (head_dim / 8) + 2 * c + m) * 64 + (p & 31) * 2 + g;
  cs[2 * f4 + e] = make_float2(cn, sn);
}

}  // namespace

extern "C" __global__ __launch_bounds__(256) void teeny_rope_table_f32(float2* cs, int n_pos,
                                                                       int head_dim,
                                                                       float ln_base) {
  rope_table(cs, n_pos, head_dim, ln_base);
}

#define TEENY_QKV_PARTS_INST(TN, T)                                                             \
  extern "C" __global__ __launch_bounds__(256) void teeny_qkv_parts_rope_split_##TN(           \
      const float* parts, int n_parts, long part_stride, T* q_out, T* k_cache, T* v_cache,      \
      int seq, const int* pos_dev, int pos0, int cache_len, int hq, int hkv, int head_dim,      \
      float ln_base) {                                                                          \
    qkv_rope_split<T, true, 4, 4>(nullptr, q_out, k_cache, v_cache, seq, pos_dev, pos0,        \
                                  cache_len, hq, hkv, head_dim, ln_base, parts, n_parts,        \
                                  part_stride);                                                 \
  }
TEENY_QKV_PARTS_INST(f32, float)
TEENY_QKV_PARTS_INST(bf16, bf16)

#define TEENY_LLAMA_INST(TN, T)                                                                 \
  extern "C" __global__ __launch_bounds__(256) void teeny_qkv_rope_split_##TN(                 \
      const T* qkv, T* q_out, T* k_cache, T* v_cache, int seq, const int* pos_dev, int pos0,    \
      int cache_len, int hq, int hkv, int head_dim, float ln_base) {                            \
    qkv_rope_rows<T>(qkv, q_out, k_cache, v_cache, seq, pos_dev, pos0, cache_len, hq, hkv,      \
                     head_dim, ln_base);                                                        \
  }                                                                                             \
  extern "C" __global__ __launch_bounds__(256) void teeny_decode_attn_partial_##TN(            \
      const T* q, const T* kc, const T* vc, float* pm, float* pl, float* po, int hq, int hkv,   \
      const int* n_past, int n_keys, int cache_len, int head_dim, float scale) {                \
    decode_partial<T>(q, kc, vc, pm, pl, po, hq, hkv, n_past, n_keys, cache_len, head_dim,      \
                      scale);                                                                   \
  }                                                                                             \
  extern "C" __global__ __launch_bounds__(256) void teeny_decode_attn_combine_##TN(            \
      const float* pm, const float* pl, const float* po, T* o, int n_chunks, int head_dim) {    \
    decode_combine<T>(pm, pl, po, o, n_chunks, head_dim);                                       \
  }                                                                                             \
  extern "C" __global__ __launch_bounds__(1024) void teeny_argmax_rows_##TN(                   \
      const T* x, long long* out, int cols) {                                                   \
    argmax_rows<T>(x, out, cols);                                                               \
  }

TEENY_LLAMA_INST(f32, float)
TEENY_LLAMA_INST(bf16, bf16)

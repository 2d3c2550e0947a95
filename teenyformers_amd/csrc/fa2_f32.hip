// fp32 flash-attention 2, forward and backward: the reference's precision.
//
// Reference: flash_attn2_causal_fwd (src/kernels/flash_attn2.rs:61-126), the
// bidirectional forward it mirrors (:57-58), flash_attn2_causal_bwd (:135-203)
// and flash_attn2_backward (:209-279).  The reference runs one 128-thread CTA
// per query row and walks every key, masked ones included, and adds dK/dV
// with fp32 atomics.  Here:
//   forward  one lane per query row, 64 rows per workgroup, K/V tiles staged
//            in LDS, the reference's per-key online-softmax update verbatim,
//            causal blocks skipped (bit-identical: a masked key is a no-op);
//   backward split like FA2's two-kernel form: a q-parallel kernel for dQ and
//            a k-parallel kernel for dK/dV (no atomics, deterministic), after
//            a preprocess that stores Delta = rowsum(O * dO).
// Layout [B, H, S, D] contiguous (= the reference's [BH, S, D]); GQA maps q
// head h to kv head h / (Hq / Hkv).
#include "common.h"

#pragma clang fp contract(off)

namespace {

constexpr int kRows = 64;  // query (or key) rows per workgroup, one per lane
constexpr int kTile = 32;  // staged rows per LDS tile

template <int D, bool CAUSAL>
__device__ void fwd_f32(const float* __restrict__ q, const float* __restrict__ k,
                        const float* __restrict__ v, float* __restrict__ o,
                        float* __restrict__ lse, int nq, int nk, float scale, int hq, int hkv) {
  __shared__ float ks[kTile][D];
  __shared__ float vs[kTile][D];
  const int bh = blockIdx.y;
  const int b = bh / hq, h = bh - b * hq;
  const long kvh = (long)b * hkv + h / (hq / hkv);
  const int qpos = blockIdx.x * kRows + threadIdx.x;
  const bool active = qpos < nq;
  const float* qrow = q + ((long)bh * nq + (active ? qpos : 0)) * D;
  const float* kb = k + kvh * (long)nk * D;
  const float* vb = v + kvh * (long)nk * D;
  float qv[D], acc[D];
#pragma unroll
  for (int j = 0; j < D; ++j) {
    qv[j] = qrow[j];
    acc[j] = 0.0f;
  }
  float m = -INFINITY, l = 0.0f;
  int kend = nk;
  if (CAUSAL) kend = min(nk, blockIdx.x * kRows + kRows);
  for (int t0 = 0; t0 < kend; t0 += kTile) {
    __syncthreads();
    for (int i = threadIdx.x; i < kTile * D; i += kRows) {
      int r = i / D, c = i - r * D;
      bool ok = t0 + r < nk;
      ks[r][c] = ok ? kb[(long)(t0 + r) * D + c] : 0.0f;
      vs[r][c] = ok ? vb[(long)(t0 + r) * D + c] : 0.0f;
    }
    __syncthreads();
    const int tn = min(kTile, kend - t0);
    for (int r = 0; r < tn; ++r) {
      const int kr = t0 + r;
      if (CAUSAL && kr > qpos) break;
      float dot = 0.0f;
#pragma unroll
      for (int j = 0; j < D; ++j) dot += qv[j] * ks[r][j];
      float s = dot * scale;
      float m_new = fmaxf(m, s);
      float e = expf(m - m_new);
      float p = expf(s - m_new);
      l = e * l + p;
#pragma unroll
      for (int j = 0; j < D; ++j) acc[j] = e * acc[j] + p * vs[r][j];
      m = m_new;
    }
  }
  if (!active) return;
  float* orow = o + ((long)bh * nq + qpos) * D;
#pragma unroll
  for (int j = 0; j < D; ++j) orow[j] = acc[j] / l;
  lse[(long)bh * nq + qpos] = m + logf(l);
}

// Delta[bh, q] = sum_d O * dO   (flash_attn2.rs:171 / :247)
template <int D>
__device__ void bwd_pre_f32(const float* __restrict__ o, const float* __restrict__ dout,
                            float* __restrict__ delta, long rows) {
  long r = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < D; ++j) s += o[r * D + j] * dout[r * D + j];
  delta[r] = s;
}

// dQ: one lane per query row, walking keys 0..q (causal) or all keys.
template <int D, bool CAUSAL>
__device__ void bwd_dq_f32(const float* __restrict__ q, const float* __restrict__ k,
                           const float* __restrict__ v, const float* __restrict__ dout,
                           const float* __restrict__ lse, const float* __restrict__ delta,
                           float* __restrict__ dq, int nq, int nk, float scale, int hq, int hkv) {
  __shared__ float ks[kTile][D];
  __shared__ float vs[kTile][D];
  const int bh = blockIdx.y;
  const int b = bh / hq, h = bh - b * hq;
  const long kvh = (long)b * hkv + h / (hq / hkv);
  const int qpos = blockIdx.x * kRows + threadIdx.x;
  const bool active = qpos < nq;
  const long row = (long)bh * nq + (active ? qpos : 0);
  const float* kb = k + kvh * (long)nk * D;
  const float* vb = v + kvh * (long)nk * D;
  float qv[D], dov[D], acc[D];
#pragma unroll
  for (int j = 0; j < D; ++j) {
    qv[j] = q[row * D + j];
    dov[j] = dout[row * D + j];
    acc[j] = 0.0f;
  }
  const float L = lse[row], Dq = delta[row];
  int kend = nk;
  if (CAUSAL) kend = min(nk, blockIdx.x * kRows + kRows);
  for (int t0 = 0; t0 < kend; t0 += kTile) {
    __syncthreads();
    for (int i = threadIdx.x; i < kTile * D; i += kRows) {
      int r = i / D, c = i - r * D;
      bool ok = t0 + r < nk;
      ks[r][c] = ok ? kb[(long)(t0 + r) * D + c] : 0.0f;
      vs[r][c] = ok ? vb[(long)(t0 + r) * D + c] : 0.0f;
    }
    __syncthreads();
    const int tn = min(kTile, kend - t0);
    for (int r = 0; r < tn; ++r) {
      const int kr = t0 + r;
      if (CAUSAL && kr > qpos) break;
      float dot = 0.0f, dpv = 0.0f;
#pragma unroll
      for (int j = 0; j < D; ++j) dot += qv[j] * ks[r][j];
#pragma unroll
      for (int j = 0; j < D; ++j) dpv += dov[j] * vs[r][j];
      float p = expf(dot * scale - L);
      float ds = p * (dpv - Dq);
#pragma unroll
      for (int j = 0; j < D; ++j) acc[j] += ds * ks[r][j] * scale;
    }
  }
  if (!active) return;
#pragma unroll
  for (int j = 0; j < D; ++j) dq[row * D + j] = acc[j];
}

// dK, dV: one lane per key row of a kv head, walking the q rows of every q
// head in its GQA group (q >= key when causal).
template <int D, bool CAUSAL>
__device__ void bwd_dkdv_f32(const float* __restrict__ q, const float* __restrict__ k,
                             const float* __restrict__ v, const float* __restrict__ dout,
                             const float* __restrict__ lse, const float* __restrict__ delta,
                             float* __restrict__ dk, float* __restrict__ dv, int nq, int nk,
                             float scale, int hq, int hkv) {
  __shared__ float qs[kTile][D];
  __shared__ float dos[kTile][D];
  __shared__ float ls[kTile], dls[kTile];
  const int kvh = blockIdx.y;  // b * hkv + hk
  const int b = kvh / hkv, hk = kvh - b * hkv;
  const int group = hq / hkv;
  const int kpos = blockIdx.x * kRows + threadIdx.x;
  const bool active = kpos < nk;
  const long krow = (long)kvh * nk + (active ? kpos : 0);
  float kv[D], vv[D], dka[D], dva[D];
#pragma unroll
  for (int j = 0; j < D; ++j) {
    kv[j] = k[krow * D + j];
    vv[j] = v[krow * D + j];
    dka[j] = 0.0f;
    dva[j] = 0.0f;
  }
  const int qstart = CAUSAL ? blockIdx.x * kRows : 0;
  for (int hh = 0; hh < group; ++hh) {
    const long bh = (long)b * hq + (long)hk * group + hh;
    for (int t0 = (qstart / kTile) * kTile; t0 < nq; t0 += kTile) {
      __syncthreads();
      for (int i = threadIdx.x; i < kTile * D; i += kRows) {
        int r = i / D, c = i - r * D;
        bool ok = t0 + r < nq;
        long qr = bh * nq + t0 + r;
        qs[r][c] = ok ? q[qr * D + c] : 0.0f;
        dos[r][c] = ok ? dout[qr * D + c] : 0.0f;
      }
      if (threadIdx.x < kTile) {
        bool ok = t0 + (int)threadIdx.x < nq;
        ls[threadIdx.x] = ok ? lse[bh * nq + t0 + threadIdx.x] : 0.0f;
        dls[threadIdx.x] = ok ? delta[bh * nq + t0 + threadIdx.x] : 0.0f;
      }
      __syncthreads();
      const int tn = min(kTile, nq - t0);
      for (int r = 0; r < tn; ++r) {
        const int qp = t0 + r;
        if (CAUSAL && kpos > qp) continue;
        float dot = 0.0f, dpv = 0.0f;
#pragma unroll
        for (int j = 0; j < D; ++j) dot += qs[r][j] * kv[j];
#pragma unroll
        for (int j = 0; j < D; ++j) dpv += dos[r][j] * vv[j];
        float p = expf(dot * scale - ls[r]);
        float ds = p * (dpv - dls[r]);
#pragma unroll
        for (int j = 0; j < D; ++j) {
          dva[j] += p * dos[r][j];
          dka[j] += ds * qs[r][j] * scale;
        }
      }
    }
  }
  if (!active) return;
#pragma unroll
  for (int j = 0; j < D; ++j) {
    dk[krow * D + j] = dka[j];
    dv[krow * D + j] = dva[j];
  }
}

}  // namespace

#define TEENY_FA2_F32_INST(D)                                                                     \
  extern "C" __global__ __launch_bounds__(64) void teeny_fa2_fwd_f32_d##D##_c(                  \
      const float* q, const float* k, const float* v, float* o, float* l, int nq, int nk,         \
      float scale, int hq, int hkv) {                                                             \
    fwd_f32<D, true>(q, k, v, o, l, nq, nk, scale, hq, hkv);                                      \
  }                                                                                               \
  extern "C" __global__ __launch_bounds__(64) void teeny_fa2_fwd_f32_d##D##_n(                  \
      const float* q, const float* k, const float* v, float* o, float* l, int nq, int nk,         \
      float scale, int hq, int hkv) {                                                             \
    fwd_f32<D, false>(q, k, v, o, l, nq, nk, scale, hq, hkv);                                     \
  }                                                                                               \
  extern "C" __global__ __launch_bounds__(256) void teeny_fa2_bwd_pre_f32_d##D(                 \
      const float* o, const float* dout, float* delta, long rows) {                               \
    bwd_pre_f32<D>(o, dout, delta, rows);                                                         \
  }                                                                                               \
  extern "C" __global__ __launch_bounds__(64) void teeny_fa2_bwd_dq_f32_d##D##_c(               \
      const float* q, const float* k, const float* v, const float* dout, const float* lse,        \
      const float* delta, float* dq, int nq, int nk, float scale, int hq, int hkv) {              \
    bwd_dq_f32<D, true>(q, k, v, dout, lse, delta, dq, nq, nk, scale, hq, hkv);                  \
  }                                                                                               \
  extern "C" __global__ __launch_bounds__(64) void teeny_fa2_bwd_dq_f32_d##D##_n(               \
      const float* q, const float* k, const float* v, const float* dout, const float* lse,        \
      const float* delta, float* dq, int nq, int nk, float scale, int hq, int hkv) {              \
    bwd_dq_f32<D, false>(q, k, v, dout, lse, delta, dq, nq, nk, scale, hq, hkv);                 \
  }                                                                                               \
  extern "C" __global__ __launch_bounds__(64) void teeny_fa2_bwd_dkdv_f32_d##D##_c(             \
      const float* q, const float* k, const float* v, const float* dout, const float* lse,        \
      const float* delta, float* dk, float* dv, int nq, int nk, float scale, int hq, int hkv) {   \
    bwd_dkdv_f32<D, true>(q, k, v, dout, lse, delta, dk, dv, nq, nk, scale, hq, hkv);            \
  }                                                                                               \
  extern "C" __global__ __launch_bounds__(64) void teeny_fa2_bwd_dkdv_f32_d##D##_n(             \
      const float* q, const float* k, const float* v, const float* dout, const float* lse,        \
      const float* delta, float* dk, float* dv, int nq, int nk, float scale, int hq, int hkv) {   \
    bwd_dkdv_f32<D, false>(q, k, v, dout, lse, delta, dk, dv, nq, nk, scale, hq, hkv);           \
  }

TEENY_FA2_F32_INST(8)
TEENY_FA2_F32_INST(16)
TEENY_FA2_F32_INST(32)
TEENY_FA2_F32_INST(64)
TEENY_FA2_F32_INST(128)

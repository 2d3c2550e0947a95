/*
 * oracle.c -- CPU restatement of teenyformers' attention hot-path kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity reference for the HIP
 * library and the timed CPU baseline.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it, and only to check results; the
 * product path (teenyformers_amd) never calls into it.
 *
 * Every function restates one reference kernel, in fp32 and in the
 * reference's per-row order, and cites the reference file:line it follows.
 * The reference is a Rust crate whose kernels are written in a Triton-like
 * DSL and compiled to PTX by an external compiler; none of it can be built
 * here, so this restatement is the oracle.
 *
 * Extensions over the reference (which has no batch dimension and no GQA):
 *   - a leading batch dimension: B independent [H, S, D] problems;
 *   - grouped-query attention: q head h reads kv head h / (Hq / Hkv).
 *   With B = 1 and Hq = Hkv these reduce to the reference exactly.
 *
 * Pinning (how each function is checked; see tests/test_oracle.py):
 *   orc_rope               reference fixture tests/golden/rope (1e-4, the
 *                          reference's own tolerance) + closed form + R(-t)R(t)=I
 *   orc_rope_at            bit-equal to orc_rope on rows padded to start at pos0,
 *                          + the float64 closed form at positions past 500
 *   orc_swiglu_fwd         reference fixture tests/golden/swiglu
 *   orc_swiglu_bwd         fp64 central finite differences
 *   orc_fused_add_rmsnorm_fwd  reference fixture tests/golden/fused_add_rmsnorm (y and h)
 *   orc_fused_add_rmsnorm_bwd  fp64 central finite differences at w == 1, and its
 *                          exact difference from orc_rmsnorm_bwd for general w
 *   orc_rmsnorm_bwd        fp64 central finite differences (dx and dw)
 *   orc_rmsnorm_fwd        closed form (generate.py:106-108) + fused kernel with r=0
 *   orc_fa2_fwd            fp64 dense softmax attention (orc_attn_dense_f64),
 *                          encoder/decoder block fixtures (attention inside a
 *                          block, RoPE off), causal row 0 == v0, convexity
 *   orc_fa2_bwd            fp64 dense analytic gradients + central finite
 *                          differences of a scalar loss through orc_fa2_fwd
 *   orc_attn_dense_f64     brute force on tiny shapes vs. numpy float64
 *   orc_transpose_heads    merge(transpose(x)) == x, brute-force index formula
 *   orc_token_embed        brute-force row gather
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define EXPORT __attribute__((visibility("default")))

EXPORT int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

EXPORT void orc_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* ------------------------------------------------------------------------ */
/* Flash attention 2 forward                                                 */
/* ------------------------------------------------------------------------ */

/*
 * One query row of flash_attn2_causal_fwd (src/kernels/flash_attn2.rs:61-126).
 *   s      = (q . k) * scale                  (:101, dot first, then x scale)
 *   mask   k_row > q_row  -> s = neg_inf      (:104-107, top-left aligned)
 *   m_new  = max(m, s); e = exp(m - m_new); p = exp(s - m_new)   (:109-111)
 *   l      = e * l + p;  acc = e * acc + p * v                   (:113-114)
 *   o      = acc / l;    lse = m + ln(l)                         (:120-122)
 * The non-causal kernel is the same loop without the mask (:57-58).
 * `all_keys` = 1 walks every key like the reference (:95); 0 stops at the
 * diagonal, which is bit-identical: a masked key leaves m, l and acc exactly
 * unchanged (e = exp(0) = 1, p = exp(-inf) = 0).
 */
static void fa2_fwd_row(const float* qrow, const float* kbase, const float* vbase,
                        float* orow, float* lse_out, int nk, int d, float scale,
                        int causal, int qpos, int all_keys, float* acc) {
  float m = -INFINITY, l = 0.0f;
  for (int j = 0; j < d; ++j) acc[j] = 0.0f;
  int kend = nk;
  if (causal && !all_keys) kend = qpos + 1 < nk ? qpos + 1 : nk;
  for (int kr = 0; kr < kend; ++kr) {
    const float* krow = kbase + (size_t)kr * d;
    const float* vrow = vbase + (size_t)kr * d;
    float dot = 0.0f;
    for (int j = 0; j < d; ++j) dot += qrow[j] * krow[j];
    float s = dot * scale;
    if (causal && kr > qpos) s = -INFINITY;
    float m_new = s > m ? s : m;
    float e = expf(m - m_new);
    float p = expf(s - m_new);
    l = e * l + p;
    for (int j = 0; j < d; ++j) acc[j] = e * acc[j] + p * vrow[j];
    m = m_new;
  }
  for (int j = 0; j < d; ++j) orow[j] = acc[j] / l;
  *lse_out = m + logf(l);
}

/*
 * q [B, Hq, Nq, D], k/v [B, Hkv, Nk, D], o [B, Hq, Nq, D], lse [B*Hq, Nq].
 * Layout [BH, N_CTX, HEAD_DIM] as in src/kernels/flash_attn2.rs:23.
 * q_offset: causal position of q row 0 (0 for a whole sequence; lets a
 * checker evaluate a slice of query rows of a long sequence).
 */
EXPORT void orc_fa2_fwd(const float* q, const float* k, const float* v, float* o, float* lse,
                        int batch, int hq, int hkv, int nq, int nk, int d, float scale,
                        int causal, int all_keys, int q_offset) {
  const int group = hq / hkv;
  const long rows = (long)batch * hq * nq;
#pragma omp parallel
  {
    float* acc = (float*)malloc(sizeof(float) * d);
#pragma omp for schedule(dynamic, 16)
    for (long r = 0; r < rows; ++r) {
      long bh = r / nq;
      int qpos = (int)(r % nq);
      int b = (int)(bh / hq), h = (int)(bh % hq);
      long kvh = (long)b * hkv + h / group;
      fa2_fwd_row(q + (size_t)r * d, k + (size_t)kvh * nk * d, v + (size_t)kvh * nk * d,
                  o + (size_t)r * d, lse + r, nk, d, scale, causal, qpos + q_offset, all_keys,
                  acc);
    }
    free(acc);
  }
}

/* ------------------------------------------------------------------------ */
/* Flash attention 2 backward                                                */
/* ------------------------------------------------------------------------ */

/*
 * flash_attn2_causal_bwd (src/kernels/flash_attn2.rs:135-203) and the
 * bidirectional flash_attn2_backward (:209-279):
 *   Dq  = sum(o * do)                                  (:171 / :247)
 *   p   = k > q ? 0 : exp(scale*(q.k) - L)             (:186-189 / :259-260)
 *   dS  = p * (do.v - Dq)                              (:191-192 / :263-264)
 *   dq += dS * k * scale                               (:194 / :267)
 *   dv[k] += p * do;  dk[k] += dS * q * scale          (:196-197 / :270-273)
 * The reference computes each (q, k) term once and adds it to dk/dv with fp32
 * atomics from every query-row CTA, so its dk/dv summation order is
 * nondeterministic.  Here the same terms are evaluated in two row-parallel
 * passes: pass 1 walks each query row's keys (dq, as the reference), pass 2
 * walks each key row's queries (q heads of the GQA group, then rows, in
 * order) and sums dk/dv deterministically.  dk/dv are overwritten, matching
 * the reference's "zero-initialised by the executor" contract (:35).
 * q_offset: causal position of q row 0 (see orc_fa2_fwd).
 */
EXPORT void orc_fa2_bwd(const float* q, const float* k, const float* v, const float* o,
                        const float* dout, const float* lse, float* dq, float* dk, float* dv,
                        int batch, int hq, int hkv, int nq, int nk, int d, float scale,
                        int causal, int all_keys, int q_offset) {
  const int group = hq / hkv;
  const long qrows = (long)batch * hq * nq;
  float* delta = (float*)malloc(sizeof(float) * (size_t)qrows);
#pragma omp parallel for schedule(dynamic, 16)
  for (long r = 0; r < qrows; ++r) {
    long bh = r / nq;
    int qp = (int)(r % nq) + q_offset;
    int b = (int)(bh / hq), h = (int)(bh % hq);
    long kvh = (long)b * hkv + h / group;
    const float* kb = k + (size_t)kvh * nk * d;
    const float* vb = v + (size_t)kvh * nk * d;
    const float* qv = q + (size_t)r * d;
    const float* dov = dout + (size_t)r * d;
    const float* ov = o + (size_t)r * d;
    float* dqv = dq + (size_t)r * d;
    float L = lse[r];
    float Dq = 0.0f;
    for (int j = 0; j < d; ++j) Dq += ov[j] * dov[j];
    delta[r] = Dq;
    for (int j = 0; j < d; ++j) dqv[j] = 0.0f;
    int kend = nk;
    if (causal && !all_keys) kend = qp + 1 < nk ? qp + 1 : nk;
    for (int kr = 0; kr < kend; ++kr) {
      const float* kv = kb + (size_t)kr * d;
      const float* vv = vb + (size_t)kr * d;
      float dot = 0.0f, dov_v = 0.0f;
      for (int j = 0; j < d; ++j) dot += qv[j] * kv[j];
      for (int j = 0; j < d; ++j) dov_v += dov[j] * vv[j];
      float p = expf(dot * scale - L);
      if (causal && kr > qp) p = 0.0f;
      float ds = p * (dov_v - Dq);
      for (int j = 0; j < d; ++j) dqv[j] += ds * kv[j] * scale;
    }
  }
  const long krows = (long)batch * hkv * nk;
#pragma omp parallel for schedule(dynamic, 16)
  for (long r = 0; r < krows; ++r) {
    long kvh = r / nk;
    int kr = (int)(r % nk);
    int b = (int)(kvh / hkv), hk = (int)(kvh % hkv);
    const float* kv = k + (size_t)r * d;
    const float* vv = v + (size_t)r * d;
    float* dkr = dk + (size_t)r * d;
    float* dvr = dv + (size_t)r * d;
    for (int j = 0; j < d; ++j) dkr[j] = dvr[j] = 0.0f;
    for (int hh = 0; hh < group; ++hh) {
      long bh = (long)b * hq + (long)hk * group + hh;
      int qstart = 0;
      if (causal && !all_keys) qstart = kr - q_offset > 0 ? kr - q_offset : 0;
      for (int qi = qstart; qi < nq; ++qi) {
        size_t row = (size_t)bh * nq + qi;
        const float* qv = q + row * d;
        const float* dov = dout + row * d;
        float dot = 0.0f, dov_v = 0.0f;
        for (int j = 0; j < d; ++j) dot += qv[j] * kv[j];
        for (int j = 0; j < d; ++j) dov_v += dov[j] * vv[j];
        float p = expf(dot * scale - lse[row]);
        if (causal && kr > qi + q_offset) p = 0.0f;
        float ds = p * (dov_v - delta[row]);
        for (int j = 0; j < d; ++j) {
          dvr[j] += p * dov[j];
          dkr[j] += ds * qv[j] * scale;
        }
      }
    }
  }
  free(delta);
}

/*
 * Textbook attention in float64, used to pin orc_fa2_fwd / orc_fa2_bwd:
 *   S = scale * Q K^T (+ causal mask k > q -> -inf), P = softmax_rows(S),
 *   O = P V, LSE = logsumexp_rows(S);
 *   given dO: dV = P^T dO, dP = dO V^T, dS = P o (dP - rowsum(dO o O)),
 *   dQ = scale dS K, dK = scale dS^T Q.
 * GQA gradients for a kv head are the sums over its q heads.
 * Inputs are fp32 (upcast); outputs are float64.  dout may be NULL.
 */
EXPORT void orc_attn_dense_f64(const float* q, const float* k, const float* v, const float* dout,
                               double* o, double* lse, double* dq, double* dk, double* dv,
                               int batch, int hq, int hkv, int nq, int nk, int d, double scale,
                               int causal) {
  const int group = hq / hkv;
  if (dout) {
    memset(dk, 0, sizeof(double) * (size_t)batch * hkv * nk * d);
    memset(dv, 0, sizeof(double) * (size_t)batch * hkv * nk * d);
  }
  double* P = (double*)malloc(sizeof(double) * (size_t)nq * nk);
  double* dS = (double*)malloc(sizeof(double) * (size_t)nq * nk);
  for (int b = 0; b < batch; ++b) {
    for (int h = 0; h < hq; ++h) {
      long bh = (long)b * hq + h;
      long kvh = (long)b * hkv + h / group;
      const float* Q = q + (size_t)bh * nq * d;
      const float* K = k + (size_t)kvh * nk * d;
      const float* V = v + (size_t)kvh * nk * d;
      double* O = o + (size_t)bh * nq * d;
      for (int i = 0; i < nq; ++i) {
        double mx = -INFINITY;
        for (int j = 0; j < nk; ++j) {
          double s = 0.0;
          for (int t = 0; t < d; ++t) s += (double)Q[(size_t)i * d + t] * (double)K[(size_t)j * d + t];
          s *= scale;
          if (causal && j > i) s = -INFINITY;
          P[(size_t)i * nk + j] = s;
          if (s > mx) mx = s;
        }
        double sum = 0.0;
        for (int j = 0; j < nk; ++j) {
          double e = exp(P[(size_t)i * nk + j] - mx);
          P[(size_t)i * nk + j] = e;
          sum += e;
        }
        for (int j = 0; j < nk; ++j) P[(size_t)i * nk + j] /= sum;
        lse[(size_t)bh * nq + i] = mx + log(sum);
        for (int t = 0; t < d; ++t) {
          double acc = 0.0;
          for (int j = 0; j < nk; ++j) acc += P[(size_t)i * nk + j] * (double)V[(size_t)j * d + t];
          O[(size_t)i * d + t] = acc;
        }
      }
      if (!dout) continue;
      const float* dO = dout + (size_t)bh * nq * d;
      double* dQ = dq + (size_t)bh * nq * d;
      double* dK = dk + (size_t)kvh * nk * d;
      double* dV = dv + (size_t)kvh * nk * d;
      for (int i = 0; i < nq; ++i) {
        double Di = 0.0;
        for (int t = 0; t < d; ++t) Di += (double)dO[(size_t)i * d + t] * O[(size_t)i * d + t];
        for (int j = 0; j < nk; ++j) {
          double dp = 0.0;
          for (int t = 0; t < d; ++t) dp += (double)dO[(size_t)i * d + t] * (double)V[(size_t)j * d + t];
          dS[(size_t)i * nk + j] = P[(size_t)i * nk + j] * (dp - Di);
        }
      }
      for (int i = 0; i < nq; ++i)
        for (int t = 0; t < d; ++t) {
          double acc = 0.0;
          for (int j = 0; j < nk; ++j) acc += dS[(size_t)i * nk + j] * (double)K[(size_t)j * d + t];
          dQ[(size_t)i * d + t] = acc * scale;
        }
      for (int j = 0; j < nk; ++j)
        for (int t = 0; t < d; ++t) {
          double ak = 0.0, av = 0.0;
          for (int i = 0; i < nq; ++i) {
            ak += dS[(size_t)i * nk + j] * (double)Q[(size_t)i * d + t];
            av += P[(size_t)i * nk + j] * (double)dO[(size_t)i * d + t];
          }
          dK[(size_t)j * d + t] += ak * scale;
          dV[(size_t)j * d + t] += av;
        }
    }
  }
  free(P);
  free(dS);
}

/* ------------------------------------------------------------------------ */
/* RoPE                                                                      */
/* ------------------------------------------------------------------------ */

/*
 * Inverse frequency of pair k, as rope_forward computes it
 * (src/kernels/rope.rs:86-93):  c = -2 * ln_base / HEAD_DIM  (fp32, in that
 * order, :88), inv = exp(fp32(k) * c).  exp is evaluated in double and
 * rounded once to fp32, i.e. the correctly rounded expf; the HIP kernels use
 * the same recipe so both sides share one table.
 */
EXPORT float orc_rope_inv_freq(int k, int d, float ln_base) {
  float c = (-2.0f * ln_base) / (float)d;
  float kc = (float)k * c;
  return (float)exp((double)kc);
}

/*
 * rope_forward (src/kernels/rope.rs:57-97) and rope_backward (:104-140) on
 * x [BH, N_CTX, HEAD_DIM]; position = row index within a BH slice (:68-71),
 * plus pos0 (0 in the reference; a KV-cached step's rows start later).
 *   fwd: y[2k] = x0 cos - x1 sin,  y[2k+1] = x0 sin + x1 cos      (:95-96)
 *   bwd: dx[2k] = dy0 cos + dy1 sin, dx[2k+1] = -dy0 sin + dy1 cos (:138-139)
 * theta = fp32(pos) * inv_freq; cos/sin are correctly rounded (double
 * evaluation rounded to fp32).
 */
EXPORT void orc_rope_at(const float* x, float* y, int bh, int n_ctx, int d, float ln_base,
                        int backward, int pos0) {
  const int half = d / 2;
  float* inv = (float*)malloc(sizeof(float) * half);
  for (int kk = 0; kk < half; ++kk) inv[kk] = orc_rope_inv_freq(kk, d, ln_base);
#pragma omp parallel for schedule(static)
  for (long r = 0; r < (long)bh * n_ctx; ++r) {
    int pos = pos0 + (int)(r % n_ctx);
    const float* xr = x + (size_t)r * d;
    float* yr = y + (size_t)r * d;
    for (int kk = 0; kk < half; ++kk) {
      float theta = (float)pos * inv[kk];
      float c = (float)cos((double)theta);
      float s = (float)sin((double)theta);
      float x0 = xr[2 * kk], x1 = xr[2 * kk + 1];
      if (!backward) {
        yr[2 * kk] = x0 * c - x1 * s;
        yr[2 * kk + 1] = x0 * s + x1 * c;
      } else {
        yr[2 * kk] = x0 * c + x1 * s;
        yr[2 * kk + 1] = -x0 * s + x1 * c;
      }
    }
  }
  free(inv);
}

EXPORT void orc_rope(const float* x, float* y, int bh, int n_ctx, int d, float ln_base,
                     int backward) {
  orc_rope_at(x, y, bh, n_ctx, d, ln_base, backward, 0);
}

/* ------------------------------------------------------------------------ */
/* Head transpose                                                            */
/* ------------------------------------------------------------------------ */

/*
 * transpose_heads (src/kernels/transpose_heads.rs:49-71):
 *   dst[h, s, d] = src[s, h*Dh + d]
 * merge_heads (:76-96): the inverse.  With a batch dimension this is
 * [B, S, H, Dh] <-> [B, H, S, Dh].  Pure byte copies (any element size).
 */
EXPORT void orc_transpose_heads(const void* src, void* dst, int batch, int seq, int heads,
                                int head_dim, int elem_bytes, int merge) {
  const size_t row = (size_t)head_dim * elem_bytes;
  const char* s = (const char*)src;
  char* t = (char*)dst;
  for (int b = 0; b < batch; ++b)
    for (int h = 0; h < heads; ++h)
      for (int p = 0; p < seq; ++p) {
        size_t bshd = (((size_t)b * seq + p) * heads + h) * row;
        size_t bhsd = (((size_t)b * heads + h) * seq + p) * row;
        if (!merge)
          memcpy(t + bhsd, s + bshd, row);
        else
          memcpy(t + bshd, s + bhsd, row);
      }
}

/* ------------------------------------------------------------------------ */
/* RMSNorm                                                                   */
/* ------------------------------------------------------------------------ */

/*
 * fused_add_rmsnorm_forward (src/kernels/fused_add_rmsnorm.rs:53-111):
 *   h = x + residual (stored, :86-88); rstd = rsqrt(sum(h^2) * (1/N) + eps)
 *   (:93-95); y = h * rstd * w (:108).
 */
EXPORT void orc_fused_add_rmsnorm_fwd(const float* x, const float* res, float* y, float* h,
                                      float* rstd, const float* w, int m, int n, float eps) {
  const float n_inv = 1.0f / (float)n;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < m; ++r) {
    const float* xr = x + (size_t)r * n;
    const float* rr = res ? res + (size_t)r * n : NULL;
    float* hr = h + (size_t)r * n;
    float sq = 0.0f;
    for (int c = 0; c < n; ++c) {
      float hv = xr[c] + (rr ? rr[c] : 0.0f);
      hr[c] = hv;
      sq += hv * hv;
    }
    float rs = 1.0f / sqrtf(sq * n_inv + eps);
    if (rstd) rstd[r] = rs;
    for (int c = 0; c < n; ++c) y[(size_t)r * n + c] = hr[c] * rs * w[c];
  }
}

/*
 * Plain RMSNorm y = x * rsqrt(mean(x^2) + eps) * w, the block's sym_rmsnorm
 * (src/layers/mod.rs:61-65, formula pinned by tests/fixtures/generate.py:106-108).
 */
EXPORT void orc_rmsnorm_fwd(const float* x, float* y, float* rstd, const float* w, int m, int n,
                            float eps) {
  const float n_inv = 1.0f / (float)n;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < m; ++r) {
    const float* xr = x + (size_t)r * n;
    float sq = 0.0f;
    for (int c = 0; c < n; ++c) sq += xr[c] * xr[c];
    float rs = 1.0f / sqrtf(sq * n_inv + eps);
    if (rstd) rstd[r] = rs;
    for (int c = 0; c < n; ++c) y[(size_t)r * n + c] = xr[c] * rs * w[c];
  }
}

/*
 * fused_add_rmsnorm_backward (src/kernels/fused_add_rmsnorm.rs:128-190):
 *   dot  = sum(dy * w * h)                                   (:166)
 *   g    = rstd * w * (dy - h * rstd^2 * dot / N)            (:170-184)
 *   dx = dres = g                                            (:185-186)
 *   dw  += dy * h * rstd summed over rows                    (:182, :187)
 * The reference updates dw with a racy load+store from every row CTA; here
 * it is the plain sum over rows, added to dw's incoming contents.
 */
EXPORT void orc_fused_add_rmsnorm_bwd(const float* dy, const float* h, float* dx, float* dres,
                                      float* dw, const float* w, const float* rstd, int m, int n) {
  const float n_inv = 1.0f / (float)n;
  for (int r = 0; r < m; ++r) {
    const float* dyr = dy + (size_t)r * n;
    const float* hr = h + (size_t)r * n;
    float rs = rstd[r];
    float dot = 0.0f;
    for (int c = 0; c < n; ++c) dot += dyr[c] * w[c] * hr[c];
    float rs2 = rs * rs;
    float sc = dot * n_inv;
    for (int c = 0; c < n; ++c) {
      float g = rs * w[c] * (dyr[c] - hr[c] * rs2 * sc);
      dx[(size_t)r * n + c] = g;
      if (dres) dres[(size_t)r * n + c] = g;
      dw[c] = dw[c] + dyr[c] * hr[c] * rs;
    }
  }
}

/*
 * Backward of the plain RMSNorm y = h * rstd * w (the block's sym_rmsnorm,
 * src/layers/mod.rs:61-65, whose backward lives in the absent teeny-core):
 * the true gradient
 *   dx = rstd * (w * dy - h * rstd^2 * sum(dy * w * h) / N),
 *   dw += sum over rows of dy * h * rstd.
 * It differs from the fused kernel's formula above (fused_add_rmsnorm.rs:184),
 * which multiplies the second term by w as well; the two agree when w == 1.
 */
EXPORT void orc_rmsnorm_bwd(const float* dy, const float* h, float* dx, float* dw,
                            const float* w, const float* rstd, int m, int n) {
  const float n_inv = 1.0f / (float)n;
  for (int r = 0; r < m; ++r) {
    const float* dyr = dy + (size_t)r * n;
    const float* hr = h + (size_t)r * n;
    float rs = rstd[r];
    float dot = 0.0f;
    for (int c = 0; c < n; ++c) dot += dyr[c] * w[c] * hr[c];
    float rs2 = rs * rs;
    float sc = dot * n_inv;
    for (int c = 0; c < n; ++c) {
      dx[(size_t)r * n + c] = rs * (w[c] * dyr[c] - hr[c] * rs2 * sc);
      dw[c] = dw[c] + dyr[c] * hr[c] * rs;
    }
  }
}

/* ------------------------------------------------------------------------ */
/* SwiGLU                                                                    */
/* ------------------------------------------------------------------------ */

/* swiglu_forward (src/kernels/swiglu.rs:56-88): out = silu(z[:, :F]) * z[:, F:]. */
EXPORT void orc_swiglu_fwd(const float* z, float* out, int m, int f) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < m; ++r) {
    const float* g = z + (size_t)r * 2 * f;
    const float* u = g + f;
    for (int c = 0; c < f; ++c) {
      float sig = 1.0f / (1.0f + expf(-g[c]));
      out[(size_t)r * f + c] = g[c] * sig * u[c];
    }
  }
}

/*
 * swiglu_backward (src/kernels/swiglu.rs:97-136):
 *   dgate = grad * up * sig * (1 + gate * (1 - sig));  dup = grad * silu(gate)
 */
EXPORT void orc_swiglu_bwd(const float* grad, const float* z, float* dz, int m, int f) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < m; ++r) {
    const float* g = z + (size_t)r * 2 * f;
    const float* u = g + f;
    const float* gr = grad + (size_t)r * f;
    float* dg = dz + (size_t)r * 2 * f;
    float* du = dg + f;
    for (int c = 0; c < f; ++c) {
      float sig = 1.0f / (1.0f + expf(-g[c]));
      float silu = g[c] * sig;
      float dsilu = sig * (1.0f + g[c] * (1.0f - sig));
      dg[c] = gr[c] * u[c] * dsilu;
      du[c] = gr[c] * silu;
    }
  }
}

/* ------------------------------------------------------------------------ */
/* Token embedding                                                           */
/* ------------------------------------------------------------------------ */

/*
 * token_embed_forward (src/kernels/token_embed.rs:38-76): out[s, :] =
 * w[ids[s], :], ids stored as f32 and converted to an integer (:53).
 */
EXPORT void orc_token_embed(const float* ids, const float* w, float* out, int seq, int d_model) {
  for (int s = 0; s < seq; ++s) {
    int id = (int)ids[s];
    memcpy(out + (size_t)s * d_model, w + (size_t)id * d_model, sizeof(float) * d_model);
  }
}

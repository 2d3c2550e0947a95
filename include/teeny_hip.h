/*
 * teeny_hip.h -- C ABI of the MI355X (gfx950) attention hot path.
 *
 * One function per op direction.  Each takes device pointers and scalars in
 * the order the reference's RuntimeOp::pack_args / pack_backward_args hands
 * them to its kernel's `entry_point` (cited per function), followed by the
 * extensions the reference lacks (batch, GQA head counts, head_dim, dtype),
 * an optional workspace, and the HIP stream all work is queued on.
 *
 * Conventions
 *   - Every pointer is device memory owned by the caller.  Work buffers are
 *     the caller's too: an entry point that needs one takes a workspace
 *     argument whose size a *_workspace_bytes query gives.  Functions never
 *     synchronise the device and return as soon as the work is queued on
 *     `stream` (0 = the null stream).
 *   - Set-up allocates, the calls after it do not: teeny_init (or the first
 *     call on a device) loads this library's code objects there, and
 *     teeny_linear_bf16 / teeny_linear_f32 create a hipBLASLt handle per
 *     device and a plan per product shape at a shape's first call (no
 *     workspace: hipBLASLt runs only algorithms that need none).  Call
 *     teeny_init and each product shape once before capturing a HIP graph.
 *   - Layouts are the reference's: attention tensors [B*H, S, D] contiguous
 *     (src/kernels/flash_attn2.rs:23), activations [rows, cols] row-major.
 *   - dtype is TEENY_F32 (the reference's type) or TEENY_BF16 (storage; all
 *     arithmetic is fp32, matrix products use bf16 MFMA with fp32 accumulate).
 *     LSE and rstd caches are always fp32.
 *   - Return 0 on success or a negative TEENY_ERR_* code; shapes and
 *     pointers are validated before anything is launched, nothing aborts.
 *   - Thread safety: every entry point is re-entrant; code objects are loaded
 *     once per device on first use (or by teeny_init) under a lock.
 */
#ifndef TEENY_HIP_H
#define TEENY_HIP_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TEENY_ABI_VERSION 1

typedef enum { TEENY_F32 = 0, TEENY_BF16 = 1, TEENY_I32 = 2 } teeny_dtype;

/* Or-ed into the dtype of a flash-attention backward (and its workspace
 * queries): with TEENY_BF16 inputs, dq, dk and dv are fp32 gradients, as the
 * reference's are (src/kernels/flash_attn2.rs:196-202): the kernels' fp32
 * accumulators are stored unrounded, and P and dS enter the matrix products
 * as two bf16 parts (hi = bf16(x), lo = bf16(x - hi)), so their operand
 * rounding falls from 2^-9 to 2^-17 relative.  Costs two more products per
 * tile in the dK/dV kernel and one in the dQ kernel.  No effect with
 * TEENY_F32. */
#define TEENY_GRAD_F32 0x100

#define TEENY_OK 0
#define TEENY_ERR_NULL_POINTER (-1)   /* a required pointer is NULL */
#define TEENY_ERR_INVALID_SHAPE (-2)  /* a size is <= 0, inconsistent, or too large */
#define TEENY_ERR_UNSUPPORTED (-3)    /* dtype / head_dim combination not built */
#define TEENY_ERR_WORKSPACE (-4)      /* workspace missing or smaller than required */
#define TEENY_ERR_HIP (-5)            /* a HIP runtime call failed (teeny_last_hip_error) */
#define TEENY_ERR_MODULE (-6)         /* code object or kernel symbol could not be loaded */
#define TEENY_ERR_INVALID_VALUE (-7)  /* a scalar argument is out of its domain */
#define TEENY_ERR_SCRATCH (-8)        /* needs more than the static scratch array (noalloc) */
#define TEENY_ERR_NOT_INITIALIZED (-9) /* teeny_init has not run on the device (noalloc) */

/* Library version, error text, last HIP error seen by this thread. */
int teeny_abi_version(void);
const char* teeny_strerror(int code);
int teeny_last_hip_error(void);

/* Load the code objects on the current device and look up the address of
 * the no-allocation backward's scratch array there.  Optional for every
 * other entry point (they load lazily); required, once per device, before
 * teeny_causal_flash_attn2_bwd_noalloc. */
int teeny_init(void);

/* Launch profiler (no counterpart in the reference, which has no tracing).
 * teeny_profile_enable(1) clears the records and brackets every following
 * launch with two hipEvents recorded on the launch's own stream;
 * teeny_profile_enable(0) stops recording.  kernel_stats synchronises on the
 * recorded events of one kernel symbol and returns its launch count and
 * summed duration; kernel_names lists the recorded symbols, one per line. */
int teeny_profile_enable(int on);
int teeny_profile_kernel_stats(const char* kernel_name, int* launches, double* total_ms);
int teeny_profile_kernel_names(char* buf, size_t buf_bytes);

/* --------------------------------------------------------------------------
 * Flash attention 2
 *
 * q [B*Hq, n_ctx_q, D], k/v [B*Hkv, n_ctx_k, D], o [B*Hq, n_ctx_q, D],
 * l (LSE cache, the RuntimeOp's param slot 0) [B*Hq, n_ctx_q] fp32.
 * LSE is natural-log in the scaled-score domain: m + ln(l)
 * (src/kernels/flash_attn2.rs:120-122).  Causal masks key > query, top-left
 * aligned (flash_attn2.rs:104-107).  q head h uses kv head h / (Hq / Hkv).
 * head_dim: fp32 8, 16, 32, 64, 128; bf16 64, 128.
 * neg_inf must be -INFINITY (the only value the reference passes,
 * flash_attn2.rs:478, :331).  softmax_scale: finite; > 0 for bf16 (the bf16
 * kernels fold the scale into the exponent after masking raw scores).
 * Backward dtype: TEENY_F32, TEENY_BF16 or TEENY_BF16 | TEENY_GRAD_F32.
 * ------------------------------------------------------------------------ */

/* Replaces CausalFlashAttn2RuntimeOp::pack_args + launch
 * (src/kernels/flash_attn2.rs:459-487): (q, k, v, o, l, n_ctx_q, n_ctx_k,
 * softmax_scale, neg_inf). */
int teeny_causal_flash_attn2_fwd(const void* q, const void* k, const void* v, void* o, float* l,
                                 int n_ctx_q, int n_ctx_k, float softmax_scale, float neg_inf,
                                 int batch, int n_heads_q, int n_heads_kv, int head_dim,
                                 int dtype, hipStream_t stream);

/* Replaces FlashAttn2RuntimeOp::pack_args + launch (flash_attn2.rs:309-340),
 * the bidirectional forward; same arguments. */
int teeny_flash_attn2_fwd(const void* q, const void* k, const void* v, void* o, float* l,
                          int n_ctx_q, int n_ctx_k, float softmax_scale, float neg_inf,
                          int batch, int n_heads_q, int n_heads_kv, int head_dim, int dtype,
                          hipStream_t stream);

/* The forward (causal or not) with MergeHeadsOp fused: o is written as
 * [B, n_ctx_q, n_heads_q * head_dim], the layout teeny_merge_heads makes of
 * the forward's [B, Hq, n_ctx_q, D] (the reference records the two ops one
 * after the other, src/layers/attention.rs:132-143); the same kernels, the
 * same output bits, one launch and one pass over O fewer.  l is [B*Hq,
 * n_ctx_q] as above.  bf16 only (TEENY_ERR_UNSUPPORTED otherwise). */
int teeny_flash_attn2_fwd_merged(const void* q, const void* k, const void* v, void* o, float* l,
                                 int n_ctx_q, int n_ctx_k, float softmax_scale, float neg_inf,
                                 int batch, int n_heads_q, int n_heads_kv, int head_dim,
                                 int dtype, int causal, hipStream_t stream);

/* The forward with its Q taken from the fused QKV projection and MergeHeadsOp
 * fused (no counterpart in the reference, which records TransposeHeadsOp +
 * RopeOp on Q, the attention op and MergeHeadsOp one after the other,
 * src/layers/attention.rs:97-143): qkv [B, n_ctx_q, (Hq + 2 Hkv) * D] as
 * teeny_qkv_rope_split takes it; the kernel rotates each q row r with the
 * (cos, sin) of position r from rope_cs (teeny_rope_table over at least
 * n_ctx_q positions rounded up to 32) as it loads it; k, v [B, Hkv, n_ctx_k,
 * D] (the cache teeny_qkv_rope_split wrote, q_out NULL); o [B, n_ctx_q,
 * Hq * D], l [B*Hq, n_ctx_q].  The same output bits as teeny_qkv_rope_split
 * into a Q buffer then teeny_flash_attn2_fwd_merged, without Q's write and
 * read.  bf16 only; rope_cs 16-byte aligned. */
int teeny_flash_attn2_fwd_qkv(const void* qkv, const float* rope_cs, const void* k, const void* v,
                              void* o, float* l, int n_ctx_q, int n_ctx_k, float softmax_scale,
                              float neg_inf, int batch, int n_heads_q, int n_heads_kv,
                              int head_dim, int dtype, int causal, hipStream_t stream);

/* (cos, sin) of RoPE's interleaved pairs at positions 0 .. n_pos-1 (n_pos a
 * multiple of 32, head_dim of 16): n_pos * head_dim fp32 values, theta =
 * fp32(pos) * fp32(exp_f64(fp32(k) * (-2 ln_rope_base / head_dim)))
 * (rope.rs:86-88), the values every rotating kernel here evaluates, in the
 * order teeny_flash_attn2_fwd_qkv loads them: pair k = 8c + 4g + 2m + e of
 * position p is floats 4 f + 2 e, +1 with f = ((p / 32) * (head_dim / 8) +
 * 2c + m) * 64 + (p % 32) * 2 + g.  No counterpart in the reference. */
int teeny_rope_table(float* cs, int n_pos, int head_dim, float ln_rope_base, hipStream_t stream);

/* Replaces CausalFlashAttn2RuntimeOp::pack_backward_args + launch
 * (flash_attn2.rs:493-529): (q, k, v, o, do, l, dq, dk, dv, n_ctx_q, n_ctx_k,
 * softmax_scale).  dq, dk and dv are overwritten: unlike the reference
 * (flash_attn2.rs:35) they need no zero initialisation.  dk/dv of a GQA kv
 * head are the sums over its q heads.  workspace: at least
 * teeny_flash_attn2_bwd_workspace_bytes(...) bytes of device memory. */
int teeny_causal_flash_attn2_bwd(const void* q, const void* k, const void* v, const void* o,
                                 const void* dout, const float* l, void* dq, void* dk, void* dv,
                                 int n_ctx_q, int n_ctx_k, float softmax_scale, int batch,
                                 int n_heads_q, int n_heads_kv, int head_dim, int dtype,
                                 void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Replaces FlashAttn2RuntimeOp::pack_backward_args + launch
 * (flash_attn2.rs:346-383), the bidirectional backward; same arguments. */
int teeny_flash_attn2_bwd(const void* q, const void* k, const void* v, const void* o,
                          const void* dout, const float* l, void* dq, void* dk, void* dv,
                          int n_ctx_q, int n_ctx_k, float softmax_scale, int batch, int n_heads_q,
                          int n_heads_kv, int head_dim, int dtype, void* workspace,
                          size_t workspace_bytes, hipStream_t stream);

/* Workspace the backward needs.  bf16: per (b, q head) and block of 32 query
 * rows, 32 values of -LSE/softmax_scale followed by 32 of -Delta (Delta =
 * rowsum(O * dO)), fp32, the last block padded; fp32: Delta [B*Hq, n_ctx_q].
 * No counterpart in the reference
 * (its executor sizes caches from RuntimeOp::param_shapes, flash_attn2.rs:449-457). */
size_t teeny_flash_attn2_bwd_workspace_bytes(int n_ctx_q, int batch, int n_heads_q, int head_dim,
                                             int dtype);
/* The workspace that also lets a causal bf16 GQA backward of 12288 or more
 * query rows with few key blocks (at most four 128-key blocks x batch x kv
 * heads per CU) and an even group (Hq / Hkv) split each group's q heads over
 * 4 dK/dV workgroups (2 if 4 does not divide the group), whose fp32 partial
 * sums a merge kernel adds in a fixed order; otherwise equal to the above.
 * With a smaller workspace such a backward runs its dK/dV in two wavefront
 * groups per workgroup instead (the form used from 2048 to 12287 query rows
 * of even groups).  No counterpart in the reference. */
size_t teeny_flash_attn2_bwd_workspace_bytes_gqa(int n_ctx_q, int n_ctx_k, int batch,
                                                 int n_heads_q, int n_heads_kv, int head_dim,
                                                 int dtype);

/* No counterpart in the reference: teeny_causal_flash_attn2_bwd for callers
 * that cannot allocate device memory (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc).  The workspace is a static device
 * array of this library, teeny_scratch_bytes() (16 MiB) per device, held until
 * the process ends; its address is looked up by teeny_init, which must have
 * run on the device (else TEENY_ERR_NOT_INITIALIZED: this entry point loads
 * and looks up nothing itself).  Problems whose
 * teeny_flash_attn2_bwd_workspace_bytes exceed it return TEENY_ERR_SCRATCH
 * (B*Hq*ceil32(n_ctx_q)*8 bytes for bf16: e.g. B8 Hq32 S4096 needs 8 MiB).
 * A GQA split runs when it fits in the array.  Calls no allocating routine
 * and may be captured in a HIP graph.  Every call on a device shares that
 * device's array: calls that overlap on one device (other streams or
 * threads) race.  Arguments otherwise as teeny_causal_flash_attn2_bwd. */
size_t teeny_scratch_bytes(void);
int teeny_causal_flash_attn2_bwd_noalloc(const void* q, const void* k, const void* v,
                                         const void* o, const void* dout, const float* l,
                                         void* dq, void* dk, void* dv, int n_ctx_q, int n_ctx_k,
                                         float softmax_scale, int batch, int n_heads_q,
                                         int n_heads_kv, int head_dim, int dtype,
                                         hipStream_t stream);

/* --------------------------------------------------------------------------
 * RoPE on x [BH, n_ctx, head_dim], interleaved pairs, position = row index.
 * Replaces RopeRtOp::pack_args (src/kernels/rope.rs:180-204): (x, y, n_ctx,
 * ln_rope_base) and pack_backward_args (:210-237): (dy, dx, n_ctx,
 * ln_rope_base).  head_dim: a power of two (the reference requires it,
 * rope.rs:56), at least 4 (fp32) or 8 (bf16).
 * In-place (y == x) is allowed.
 * ------------------------------------------------------------------------ */
int teeny_rope_fwd(const void* x, void* y, int n_ctx, float ln_rope_base, int bh, int head_dim,
                   int dtype, hipStream_t stream);
int teeny_rope_bwd(const void* dy, void* dx, int n_ctx, float ln_rope_base, int bh, int head_dim,
                   int dtype, hipStream_t stream);

/* --------------------------------------------------------------------------
 * Head transposes, byte-exact.
 * transpose_heads: src [B, S, H*Dh] -> dst [B, H, S, Dh].  Replaces
 *   TransposeHeads RuntimeOp::pack_args (src/kernels/transpose_heads.rs:106-129):
 *   (src, dst, seq_len, n_heads).
 * merge_heads: src [B, H, S, Dh] -> dst [B, S, H*Dh].  Replaces MergeHeads
 *   RuntimeOp::pack_args (transpose_heads.rs:214-237).
 * Each is the other's backward (transpose_heads.rs:146-154, :256-264).
 * ------------------------------------------------------------------------ */
int teeny_transpose_heads(const void* src, void* dst, int seq_len, int n_heads, int batch,
                          int head_dim, int dtype, hipStream_t stream);
int teeny_merge_heads(const void* src, void* dst, int seq_len, int n_heads, int batch,
                      int head_dim, int dtype, hipStream_t stream);

/* --------------------------------------------------------------------------
 * Fused residual add + RMSNorm over rows of N.
 * fwd replaces FusedAddRmsnormRtOp::pack_args (src/kernels/fused_add_rmsnorm.rs:227-254):
 *   (x, residual, y, h, rstd, weight, M, N, eps); h = x + residual (param
 *   slot 1), rstd [M] fp32 (param slot 2), weight [N] (slot 0).
 * bwd replaces pack_backward_args (fused_add_rmsnorm.rs:260-291):
 *   (dy, h, dx, dresidual, dweight, weight, rstd, M, N); dweight is
 *   ACCUMULATED into (dweight += sum over rows), as in the reference
 *   (fused_add_rmsnorm.rs:187), but deterministically.  dresidual may be NULL.
 *   workspace: teeny_fused_add_rmsnorm_bwd_workspace_bytes(M, N).
 * rmsnorm_fwd: the plain norm the Llama block records (src/layers/mod.rs:61-65);
 *   rstd may be NULL.
 * rmsnorm_bwd: backward of that plain norm with the true gradient
 *   dx = rstd * (w * dy - x * rstd^2 * sum(dy * w * x) / N); dweight accumulated
 *   as above; same workspace.  The fused backward keeps the reference's
 *   formula rstd * w * (dy - h * rstd^2 * sum(dy * w * h) / N)
 *   (fused_add_rmsnorm.rs:184), which equals the true gradient only when
 *   w == 1.  No reference entry point (the block's norm is teeny-core's
 *   RmsNorm, src/layers/mod.rs:61-65, whose source is absent).
 * N: a multiple of 8 (bf16) / 4 (fp32) up to 64*8*16, or any N up to 1024.
 * ------------------------------------------------------------------------ */
int teeny_fused_add_rmsnorm_fwd(const void* x, const void* residual, void* y, void* h,
                                float* rstd, const void* weight, int M, int N, float eps,
                                int dtype, hipStream_t stream);
int teeny_fused_add_rmsnorm_bwd(const void* dy, const void* h, void* dx, void* dresidual,
                                void* dweight, const void* weight, const float* rstd, int M,
                                int N, int dtype, void* workspace, size_t workspace_bytes,
                                hipStream_t stream);
size_t teeny_fused_add_rmsnorm_bwd_workspace_bytes(int M, int N);
int teeny_rmsnorm_fwd(const void* x, void* y, float* rstd, const void* weight, int M, int N,
                      float eps, int dtype, hipStream_t stream);
int teeny_rmsnorm_bwd(const void* dy, const void* x, void* dx, void* dweight, const void* weight,
                      const float* rstd, int M, int N, int dtype, void* workspace,
                      size_t workspace_bytes, hipStream_t stream);

/* --------------------------------------------------------------------------
 * SwiGLU: z [M, 2*d_ff] (gate || up) -> out [M, d_ff].
 * fwd replaces SwigluForward RuntimeOp::pack_args (src/kernels/swiglu.rs:151-173):
 *   (z, out, M, d_ff); bwd replaces pack_backward_args (:179-207):
 *   (grad, z, dz, M, d_ff).
 * ------------------------------------------------------------------------ */
int teeny_swiglu_fwd(const void* z, void* out, int M, int d_ff, int dtype, hipStream_t stream);
int teeny_swiglu_bwd(const void* grad, const void* z, void* dz, int M, int d_ff, int dtype,
                     hipStream_t stream);

/* Elementwise residual add y = a + b over n values (a, b, y 16-byte
 * aligned; y may alias a or b).  Replaces the Op::Add that sym_add records
 * (src/layers/mod.rs:36-48), which the reference lowers through teeny-core. */
int teeny_add(const void* a, const void* b, void* y, long n, int dtype, hipStream_t stream);

/* --------------------------------------------------------------------------
 * Token embedding gather: out[s, :] = weight[ids[s], :].
 * Replaces TokenEmbedRuntimeOp::pack_args (src/layers/embedding.rs:65-80):
 *   (ids, weight, out, seq_len, d_model).  ids_dtype TEENY_F32 (the
 *   reference's encoding, src/kernels/token_embed.rs:32) or TEENY_I32; an id
 *   outside [0, vocab_size) gives a zero row.
 * ------------------------------------------------------------------------ */
int teeny_token_embed_fwd(const void* ids, const void* weight, void* out, int seq_len,
                          int d_model, int vocab_size, int ids_dtype, int dtype,
                          hipStream_t stream);

/* --------------------------------------------------------------------------
 * Llama attention plumbing (extensions; no single reference op).
 *
 * teeny_qkv_rope_split: the fused QKV projection output qkv
 *   [B, seq_len, (Hq + 2*Hkv) * D] -> q_out [B, Hq, seq_len, D] with RoPE,
 *   and K (with RoPE) / V written into caches [B, Hkv, cache_len, D] at rows
 *   pos0 .. pos0+seq_len-1; RoPE positions are absolute (pos0 + s).  Fuses
 *   the reference's TransposeHeadsOp x3 + RopeOp x2 (src/layers/attention.rs:97-123)
 *   with their arithmetic (transpose_heads.rs:65-67, rope.rs:86-96).  q_out
 *   may be NULL: then only the cache rows are written (the prompt attention
 *   teeny_flash_attn2_fwd_qkv reads and rotates Q itself).
 * teeny_decode_attention: one query row per (b, q head), q [B, Hq, D],
 *   against cache rows 0 .. n_keys-1 (all visible: the newest query is the
 *   last position), o [B, Hq, D].  Split over the keys; workspace of
 *   teeny_decode_attention_workspace_bytes(...) bytes.  The reference
 *   recomputes the prefix instead (examples/llama_generate.rs:373-381).
 *   head_dim: a power of two from 8 to 128; Hq / Hkv <= 16.
 * ------------------------------------------------------------------------ */
int teeny_qkv_rope_split(const void* qkv, void* q_out, void* k_cache, void* v_cache, int batch,
                         int seq_len, int pos0, int cache_len, int n_heads_q, int n_heads_kv,
                         int head_dim, float ln_rope_base, int dtype, hipStream_t stream);
size_t teeny_decode_attention_workspace_bytes(int batch, int n_heads_q, int n_keys,
                                              int head_dim);
int teeny_decode_attention(const void* q, const void* k_cache, const void* v_cache, void* o,
                           int batch, int n_heads_q, int n_heads_kv, int n_keys, int cache_len,
                           int head_dim, float softmax_scale, int dtype, void* workspace,
                           size_t workspace_bytes, hipStream_t stream);

/* Device-position variants for a decode step captured once in a HIP graph
 * and replayed while the position advances (the reference has no KV cache
 * and no graphs; these have no counterpart there).
 * teeny_qkv_rope_split_dev: as teeny_qkv_rope_split with pos0 read from
 *   device memory (*pos0) when the kernel runs; cache rows outside
 *   [0, cache_len) are not written.
 * teeny_decode_attention_dev: as teeny_decode_attention attending to the
 *   first min(*n_past + 1, max_keys) cache rows, *n_past read when the kernel
 *   runs; the grid and the workspace are sized for max_keys
 *   (teeny_decode_attention_workspace_bytes(batch, n_heads_q, max_keys, D)). */
int teeny_qkv_rope_split_dev(const void* qkv, void* q_out, void* k_cache, void* v_cache,
                             int batch, int seq_len, const int32_t* pos0, int cache_len,
                             int n_heads_q, int n_heads_kv, int head_dim, float ln_rope_base,
                             int dtype, hipStream_t stream);
int teeny_decode_attention_dev(const void* q, const void* k_cache, const void* v_cache, void* o,
                               int batch, int n_heads_q, int n_heads_kv, const int32_t* n_past,
                               int max_keys, int cache_len, int head_dim, float softmax_scale,
                               int dtype, void* workspace, size_t workspace_bytes,
                               hipStream_t stream);

/* Row argmax of x [rows, cols] -> out[rows] (int64): the reference's greedy
 * choice (examples/llama_generate.rs:252-257), the LAST index among equal
 * maxima (Rust's Iterator::max_by); NaN, on which the reference's comparison
 * panics, counts as the maximum (the last NaN wins). */
int teeny_argmax_rows(const void* x, int64_t* out, int rows, int cols, int dtype,
                      hipStream_t stream);

/* Linear layer y[M, N] = x[M, K] . w[N, K]^T in bf16, any M >= 1: replaces
 * the external teeny-core Linear behind sym_linear (src/layers/mod.rs:54-58).
 * Up to 16 rows (a KV-cached decode step) with N % 128 == 0 and K % 128 == 0
 * stream the weight through a GEMV-shaped kernel; more rows go to hipBLASLt
 * (faster than this library's GEMM at the Llama prompt shapes), and to
 * teeny_gemm_bf16 where hipBLASLt does not take the device or shape or the
 * stream is capturing (a fixed rule: a captured product never runs
 * hipBLASLt); both require N % 64 == 0 and K % 64 == 0 (otherwise
 * TEENY_ERR_UNSUPPORTED).  Every path accumulates in fp32 and rounds each
 * output to bf16 once; none uses a workspace.
 * teeny_linear_swiglu_bf16: w is the fused gate_up weight [2F, K] (gate rows
 * first, src/loader.rs:49-55); writes y[M, F] = silu(x w_gate^T) *
 * (x w_up^T) with both products rounded to bf16 first, as FeedForward's
 * gate_up Linear followed by SwigluOp computes it (src/layers/ffn.rs:47-56),
 * without writing the [M, 2F] product: up to 16 rows with F % 64 == 0 and
 * K % 128 == 0 take the weight-streaming kernel, other shapes the GEMM with
 * the SwiGLU in its epilogue (F % 32 == 0 and K % 64 == 0, otherwise
 * TEENY_ERR_UNSUPPORTED).  Bit-identical to teeny_linear_bf16 on [2F, K]
 * followed by teeny_swiglu_fwd. */
int teeny_linear_bf16(const void* x, const void* w, void* y, int M, int N, int K,
                      hipStream_t stream);
/* This library's matrix-core GEMM for the same product, any M (N and K
 * multiples of 64): teeny_linear_bf16's fallback above 16 rows, and the
 * kernel whose epilogue forms teeny_linear_swiglu_bf16 at those sizes. */
int teeny_gemm_bf16(const void* x, const void* w, void* y, int M, int N, int K,
                    hipStream_t stream);
int teeny_linear_swiglu_bf16(const void* x, const void* w, void* y, int M, int F, int K,
                             hipStream_t stream);

/* The same Linear in fp32, the reference's precision (teeny-core's Linear
 * behind sym_linear, src/layers/mod.rs:54-58, on the f32 weights that
 * src/loader.rs:41,66-80 decodes): hipBLASLt's fp32 GEMM (fp32 products
 * and accumulation, no workspace), or teeny_gemm_f32 where hipBLASLt does
 * not take the device or shape or the stream is capturing.  Any M and N; K
 * a multiple of 4; x and w 16-byte aligned. */
int teeny_linear_f32(const void* x, const void* w, void* y, int M, int N, int K,
                     hipStream_t stream);
/* This library's fp32 GEMM for the same product: each output one fp32
 * fused multiply-add chain over k in increasing order. */
int teeny_gemm_f32(const void* x, const void* w, void* y, int M, int N, int K,
                   hipStream_t stream);

/* The same product split over K for more parallelism at small N: writes
 * teeny_linear_partials_count(K, k_split) fp32 slabs parts[n][M][N], slab i
 * summing k in [i k_split, (i+1) k_split).  k_split is a multiple of 128 or
 * >= K.  The slabs are consumed, summed in slab order and rounded to the
 * activation dtype (as the unsplit product would be stored), by
 * teeny_fused_add_rmsnorm_partials_fwd (x = the sum; otherwise as
 * teeny_fused_add_rmsnorm_fwd, src/kernels/fused_add_rmsnorm.rs:53-110) and
 * teeny_qkv_rope_split_partials_dev (qkv = the sum; otherwise as
 * teeny_qkv_rope_split_dev).  No reference counterpart: the reference has no
 * decode path with a KV cache. */
int teeny_linear_partials_count(int K, int k_split);
int teeny_linear_partials_bf16(const void* x, const void* w, float* parts, int M, int N, int K,
                               int k_split, hipStream_t stream);

/* The streaming layout of a bf16 weight W [N, K] (row-major, the HF [out,
 * in] layout of src/loader.rs:19-27) for the decode-step kernels: a copy
 * w_s of N*K bf16 in the order their wavefronts load it,
 *   w_s[nb][ks][q][g][r][e] = W[16 nb + r][128 ks + 32 g + 8 q + e]
 * (nb < N/16, ks < K/128, q, g < 4, r < 16, e < 8), so that each load
 * instruction reads one contiguous KiB.  N % 16 == 0 and K % 128 == 0
 * (TEENY_ERR_UNSUPPORTED otherwise); w and w_s must not overlap
 * (TEENY_ERR_INVALID_VALUE).  Done once per weight, at load time.
 * teeny_linear_sl_bf16, teeny_linear_swiglu_sl_bf16 (w_s: the layout of the
 * fused [2F, K] gate_up weight) and teeny_linear_partials_sl_bf16 are
 * teeny_linear_bf16, teeny_linear_swiglu_bf16 and teeny_linear_partials_bf16
 * at up to 16 rows (M <= 16, N % 128 == 0 or F % 64 == 0, K % 128 == 0;
 * TEENY_ERR_UNSUPPORTED otherwise) reading W from w_s: the same products in
 * the same order, bit-identical outputs, in 3-9 % less time on weights that
 * stream from HBM.  No reference counterpart: a layout for this library's
 * decode kernels, costing one more copy of the weights they read. */
int teeny_linear_stream_layout_bf16(const void* w, void* w_s, int N, int K, hipStream_t stream);
int teeny_linear_sl_bf16(const void* x, const void* w_s, void* y, int M, int N, int K,
                         hipStream_t stream);
int teeny_linear_swiglu_sl_bf16(const void* x, const void* w_s, void* y, int M, int F, int K,
                                hipStream_t stream);
int teeny_linear_partials_sl_bf16(const void* x, const void* w_s, float* parts, int M, int N,
                                  int K, int k_split, hipStream_t stream);
int teeny_fused_add_rmsnorm_partials_fwd(const float* parts, int n_parts, const void* residual,
                                         void* y, void* h, float* rstd, const void* weight,
                                         int M, int N, float eps, int dtype,
                                         hipStream_t stream);
int teeny_qkv_rope_split_partials_dev(const float* parts, int n_parts, void* q_out,
                                      void* k_cache, void* v_cache, int batch, int seq_len,
                                      const int32_t* pos0, int cache_len, int n_heads_q,
                                      int n_heads_kv, int head_dim, float ln_rope_base,
                                      int dtype, hipStream_t stream);

/* teeny_decode_qkv_attention_dev: a one-token decode step's attention in
 * one launch, for position p = *n_past (read when the kernel runs): the
 * QKV projection's K-split slabs parts[n_parts][batch][(Hq + 2 Hkv) D] are
 * summed and rounded as by teeny_qkv_rope_split_partials_dev, k and v (k
 * with RoPE) are written to cache row p when p < cache_len, and q (RoPE)
 * attends to cache rows 0 .. min(p + 1, cache_len) - 1 as by
 * teeny_decode_attention_dev; o [batch, Hq, D].  bf16, D 64 or 128,
 * Hq / Hkv <= 32; no workspace.  One workgroup per (b, kv head) reads that
 * head's rows, so it suits caches of a few thousand rows; longer ones
 * spread better over the split-K teeny_decode_attention_dev.  No reference
 * counterpart (the reference has no KV cache). */
int teeny_decode_qkv_attention_dev(const float* parts, int n_parts, void* k_cache,
                                   void* v_cache, void* o, int batch, int n_heads_q,
                                   int n_heads_kv, int head_dim, int cache_len,
                                   const int32_t* n_past, float ln_rope_base,
                                   float softmax_scale, int dtype, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TEENY_HIP_H */

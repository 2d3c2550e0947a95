"""Functional API over torch tensors; every op runs the HIP kernels through
the C ABI (include/teeny_hip.h).  torch only supplies device memory and the
current stream.

Shapes follow the reference with the batch split out:
  attention tensors  [B, H, S, D]   (reference [BH, S, D], flash_attn2.rs:23)
  activations        [..., N]       (rows x columns)
"""
from __future__ import annotations

import contextlib
import math
import threading

import torch

from . import _lib
from ._lib import TEENY_BF16, TEENY_F32, TEENY_I32, call

_DTYPES = {torch.float32: TEENY_F32, torch.bfloat16: TEENY_BF16}


def _code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected float32 or bfloat16") from None


def _dev(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("teenyformers_amd ops take device tensors (no CPU fallback)")
        if not t.is_contiguous():
            raise ValueError("teenyformers_amd ops take contiguous tensors")


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _p(t):
    return None if t is None else t.data_ptr()


def _as4(x: torch.Tensor) -> torch.Tensor:
    """[BH, S, D] -> [1, BH, S, D]; [B, H, S, D] unchanged."""
    if x.dim() == 3:
        return x.unsqueeze(0)
    if x.dim() != 4:
        raise ValueError(f"attention tensors are [B, H, S, D] or [BH, S, D], got {tuple(x.shape)}")
    return x


# ---------------------------------------------------------------------------
# Flash attention 2
# ---------------------------------------------------------------------------

def flash_attn2_fwd(q, k, v, softmax_scale: float | None = None, causal: bool = True,
                    out: torch.Tensor | None = None, lse: torch.Tensor | None = None):
    """O = softmax(scale Q K^T [+ causal]) V and LSE (fp32, natural log).

    q [B, Hq, Sq, D], k/v [B, Hkv, Sk, D] (or [BH, S, D]).  Returns (o, lse)
    with lse [B, Hq, Sq].
    """
    q4, k4, v4 = _as4(q), _as4(k), _as4(v)
    _dev(q4, k4, v4)
    B, Hq, Sq, D = q4.shape
    Hkv, Sk = k4.shape[1], k4.shape[2]
    if k4.shape != v4.shape or k4.shape[0] != B or k4.shape[3] != D:
        raise ValueError("k and v must be [B, Hkv, Sk, D] matching q")
    if q4.dtype != k4.dtype or q4.dtype != v4.dtype:
        raise TypeError("q, k, v must share a dtype")
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    if out is None:
        out = torch.empty_like(q)
    if lse is None:
        lse = torch.empty((B, Hq, Sq), dtype=torch.float32, device=q.device)
    _dev(out, lse)
    fn = "teeny_causal_flash_attn2_fwd" if causal else "teeny_flash_attn2_fwd"
    call(fn, _p(q4), _p(k4), _p(v4), _p(out), _p(lse), Sq, Sk, scale, float("-inf"),
         B, Hq, Hkv, D, _code(q4), _stream())
    return out, lse


def flash_attn2_fwd_merged(q, k, v, softmax_scale: float | None = None, causal: bool = True):
    """The forward with the heads merged (MergeHeadsOp fused): o [B, Sq, Hq*D]
    (merge_heads of flash_attn2_fwd's o, bit for bit) and lse [B, Hq, Sq].
    bf16 q [B, Hq, Sq, D], k/v [B, Hkv, Sk, D]."""
    q4, k4, v4 = _as4(q), _as4(k), _as4(v)
    _dev(q4, k4, v4)
    B, Hq, Sq, D = q4.shape
    Hkv, Sk = k4.shape[1], k4.shape[2]
    if k4.shape != v4.shape or k4.shape[0] != B or k4.shape[3] != D:
        raise ValueError("k and v must be [B, Hkv, Sk, D] matching q")
    if not (q4.dtype == k4.dtype == v4.dtype == torch.bfloat16):
        raise TypeError("flash_attn2_fwd_merged: bf16 q, k, v")
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    out = torch.empty((B, Sq, Hq * D), dtype=q4.dtype, device=q4.device)
    lse = torch.empty((B, Hq, Sq), dtype=torch.float32, device=q4.device)
    call("teeny_flash_attn2_fwd_merged", _p(q4), _p(k4), _p(v4), _p(out), _p(lse), Sq, Sk, scale,
         float("-inf"), B, Hq, Hkv, D, _code(q4), int(bool(causal)), _stream())
    return out, lse


def rope_table(n_pos: int, head_dim: int, rope_base: float, device) -> torch.Tensor:
    """(cos, sin) of RoPE's pairs at positions 0 .. n_pos-1 (rounded up to 32)
    in the order flash_attn2_fwd_qkv loads them (teeny_rope_table): a flat
    fp32 tensor of n_pos * head_dim values; rope_table_pairs gives the
    [n_pos, D/2, 2] view."""
    n = (n_pos + 31) // 32 * 32
    cs = torch.empty(n * head_dim, dtype=torch.float32, device=device)
    call("teeny_rope_table", _p(cs), n, head_dim, _ln(rope_base), _stream())
    return cs


def rope_table_pairs(cs: torch.Tensor, head_dim: int) -> torch.Tensor:
    """[n_pos, D/2, 2] (cos, sin) of a rope_table: pair k = 8c + 4g + 2m + e of
    position p sits in float4 ((p/32) (D/8) + 2c + m) 64 + (p%32) 2 + g."""
    D = head_dim
    t = cs.view(-1, D // 8, 32, 2, 2, 2)      # [p/32, i = 2c + m, p%32, g, e, (cos, sin)]
    t = t.view(-1, D // 16, 2, 32, 2, 2, 2)   # [p/32, c, m, p%32, g, e, cs]
    t = t.permute(0, 3, 1, 4, 2, 5, 6)        # [p/32, p%32, c, g, m, e, cs]
    return t.reshape(-1, D // 2, 2)


def flash_attn2_fwd_qkv(qkv, rope_cs, k, v, n_heads_q: int, softmax_scale: float | None = None,
                        causal: bool = True):
    """The prompt attention straight from the fused QKV projection: qkv
    [B, S, (Hq+2Hkv)*D] bf16 (its q heads rotated as they load, row r at
    position r with rope_cs row r), k/v [B, Hkv, Sk, D] (the cache);
    returns o [B, S, Hq*D] (merged heads) and lse [B, Hq, S]."""
    _dev(qkv, rope_cs, k, v)
    B, S, W = qkv.shape
    _, Hkv, Sk, D = k.shape
    Hq = n_heads_q
    if W != (Hq + 2 * Hkv) * D or v.shape != k.shape or k.shape[0] != B:
        raise ValueError("qkv must be [B, S, (Hq+2Hkv)*D] matching k, v [B, Hkv, Sk, D]")
    if not (qkv.dtype == k.dtype == v.dtype == torch.bfloat16):
        raise TypeError("flash_attn2_fwd_qkv: bf16 qkv, k, v")
    if rope_cs.dtype != torch.float32 or rope_cs.numel() < (S + 31) // 32 * 32 * D:
        raise ValueError("rope_cs: a rope_table of at least S positions")
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    out = torch.empty((B, S, Hq * D), dtype=qkv.dtype, device=qkv.device)
    lse = torch.empty((B, Hq, S), dtype=torch.float32, device=qkv.device)
    call("teeny_flash_attn2_fwd_qkv", _p(qkv), _p(rope_cs), _p(k), _p(v), _p(out), _p(lse), S, Sk,
         scale, float("-inf"), B, Hq, Hkv, D, _code(qkv), int(bool(causal)), _stream())
    return out, lse


def flash_attn2_bwd_workspace_bytes(q: torch.Tensor, k: torch.Tensor | None = None) -> int:
    """Backward workspace; given k, the size that also allows the GQA head
    split of the dK/dV kernel where it applies."""
    q4 = _as4(q)
    B, Hq, Sq, D = q4.shape
    if k is None:
        return _lib.lib().teeny_flash_attn2_bwd_workspace_bytes(Sq, B, Hq, D, _code(q4))
    k4 = _as4(k)
    return _lib.lib().teeny_flash_attn2_bwd_workspace_bytes_gqa(Sq, k4.shape[2], B, Hq, k4.shape[1],
                                                                D, _code(q4))


def flash_attn2_bwd(q, k, v, o, lse, do, softmax_scale: float | None = None, causal: bool = True,
                    workspace: torch.Tensor | None = None, dq=None, dk=None, dv=None,
                    grad_f32: bool = False):
    """Gradients (dq, dk, dv) of sum(O * dO); dk/dv summed over each GQA group.

    grad_f32: with bf16 inputs, return fp32 gradients (the kernels' fp32
    accumulators, unrounded; TEENY_GRAD_F32)."""
    q4, k4, v4, o4, do4 = _as4(q), _as4(k), _as4(v), _as4(o), _as4(do)
    _dev(q4, k4, v4, o4, do4, lse)
    B, Hq, Sq, D = q4.shape
    Hkv, Sk = k4.shape[1], k4.shape[2]
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    ws_bytes = flash_attn2_bwd_workspace_bytes(q4, k4)
    if workspace is None:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    code = _code(q4)
    gdt = q.dtype
    if grad_f32 and q.dtype == torch.bfloat16:
        code |= _lib.TEENY_GRAD_F32
        gdt = torch.float32
    dq = torch.empty(q.shape, dtype=gdt, device=q.device) if dq is None else dq
    dk = torch.empty(k.shape, dtype=gdt, device=q.device) if dk is None else dk
    dv = torch.empty(v.shape, dtype=gdt, device=q.device) if dv is None else dv
    for g in (dq, dk, dv):
        if g.dtype != gdt or not g.is_contiguous():
            raise ValueError(f"gradient outputs must be contiguous {gdt}")
    fn = "teeny_causal_flash_attn2_bwd" if causal else "teeny_flash_attn2_bwd"
    call(fn, _p(q4), _p(k4), _p(v4), _p(o4), _p(do4), _p(lse), _p(dq), _p(dk), _p(dv),
         Sq, Sk, scale, B, Hq, Hkv, D, code, _p(workspace), workspace.numel(), _stream())
    return dq, dk, dv


class FlashAttn2Function(torch.autograd.Function):
    """Autograd wrapper: forward saves (q, k, v, o, lse) like the reference's
    LSE param cache (flash_attn2.rs:449-457) and backward recomputes P."""

    @staticmethod
    def forward(ctx, q, k, v, softmax_scale, causal):
        o, lse = flash_attn2_fwd(q, k, v, softmax_scale, causal)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.scale, ctx.causal = softmax_scale, causal
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse = ctx.saved_tensors
        dq, dk, dv = flash_attn2_bwd(q, k, v, o, lse, do.contiguous(), ctx.scale, ctx.causal)
        return dq, dk, dv, None, None


def flash_attn2(q, k, v, softmax_scale=None, causal=True):
    return FlashAttn2Function.apply(q, k, v, softmax_scale, causal)


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------

def rope(x: torch.Tensor, rope_base: float, backward: bool = False,
         out: torch.Tensor | None = None) -> torch.Tensor:
    """Interleaved-pair rotary embedding on x [..., S, D]; position = S index."""
    _dev(x)
    S, D = x.shape[-2], x.shape[-1]
    bh = x.numel() // (S * D)
    ln_base = float(torch.tensor(rope_base, dtype=torch.float32).log().item())
    out = torch.empty_like(x) if out is None else out
    _dev(out)
    fn = "teeny_rope_bwd" if backward else "teeny_rope_fwd"
    call(fn, _p(x), _p(out), S, ln_base, bh, D, _code(x), _stream())
    return out


class RopeFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, rope_base):
        ctx.rope_base = rope_base
        return rope(x, rope_base)

    @staticmethod
    def backward(ctx, dy):
        return rope(dy.contiguous(), ctx.rope_base, backward=True), None


# ---------------------------------------------------------------------------
# Head transposes
# ---------------------------------------------------------------------------

def transpose_heads(x: torch.Tensor, n_heads: int) -> torch.Tensor:
    """[B, S, H*Dh] (or [S, H*Dh]) -> [B, H, S, Dh] (or [H, S, Dh])."""
    _dev(x)
    squeeze = x.dim() == 2
    x3 = x.unsqueeze(0) if squeeze else x
    B, S, HD = x3.shape
    if HD % n_heads:
        raise ValueError("last dim must be n_heads * head_dim")
    Dh = HD // n_heads
    out = torch.empty((B, n_heads, S, Dh), dtype=x.dtype, device=x.device)
    call("teeny_transpose_heads", _p(x3), _p(out), S, n_heads, B, Dh, _code(x), _stream())
    return out[0] if squeeze else out


def merge_heads(x: torch.Tensor) -> torch.Tensor:
    """[B, H, S, Dh] (or [H, S, Dh]) -> [B, S, H*Dh] (or [S, H*Dh])."""
    _dev(x)
    squeeze = x.dim() == 3
    x4 = x.unsqueeze(0) if squeeze else x
    B, H, S, Dh = x4.shape
    out = torch.empty((B, S, H * Dh), dtype=x.dtype, device=x.device)
    call("teeny_merge_heads", _p(x4), _p(out), S, H, B, Dh, _code(x), _stream())
    return out[0] if squeeze else out


class TransposeHeadsFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, n_heads):
        return transpose_heads(x, n_heads)

    @staticmethod
    def backward(ctx, dy):
        return merge_heads(dy.contiguous()), None


class MergeHeadsFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        ctx.n_heads = x.shape[-3]
        return merge_heads(x)

    @staticmethod
    def backward(ctx, dy):
        return transpose_heads(dy.contiguous(), ctx.n_heads)


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------

def _rows(x: torch.Tensor):
    N = x.shape[-1]
    return x.numel() // N, N


def fused_add_rmsnorm(x, residual, weight, eps: float):
    """h = x + residual; y = h * rsqrt(mean(h^2) + eps) * weight -> (y, h, rstd).
    x may be Partials (summed and rounded to residual's dtype first)."""
    if isinstance(x, Partials):
        _dev(x.slabs, residual, weight)
        M, N = _rows(residual)
        if x.slabs.shape[1:] != (M, N) or x.dtype != residual.dtype:
            raise ValueError("fused_add_rmsnorm: partial slabs do not match the residual")
        y = torch.empty_like(residual)
        h = torch.empty_like(residual)
        rstd = torch.empty(M, dtype=torch.float32, device=residual.device)
        call("teeny_fused_add_rmsnorm_partials_fwd", _p(x.slabs), x.n, _p(residual), _p(y),
             _p(h), _p(rstd), _p(weight), M, N, float(eps), _code(residual), _stream())
        return y, h, rstd
    _dev(x, residual, weight)
    M, N = _rows(x)
    y = torch.empty_like(x)
    h = torch.empty_like(x)
    rstd = torch.empty(M, dtype=torch.float32, device=x.device)
    call("teeny_fused_add_rmsnorm_fwd", _p(x), _p(residual), _p(y), _p(h), _p(rstd), _p(weight),
         M, N, float(eps), _code(x), _stream())
    return y, h, rstd


def rmsnorm(x, weight, eps: float, want_rstd: bool = True):
    _dev(x, weight)
    M, N = _rows(x)
    y = torch.empty_like(x)
    rstd = torch.empty(M, dtype=torch.float32, device=x.device) if want_rstd else None
    call("teeny_rmsnorm_fwd", _p(x), _p(y), _p(rstd), _p(weight), M, N, float(eps), _code(x),
         _stream())
    return y, rstd


def _norm_ws(M, N, device):
    return torch.empty(_lib.lib().teeny_fused_add_rmsnorm_bwd_workspace_bytes(M, N),
                       dtype=torch.uint8, device=device)


def fused_add_rmsnorm_bwd(dy, h, weight, rstd, dweight=None, want_dres: bool = True):
    """The reference's fused backward (fused_add_rmsnorm.rs:128-190) -> (dx, dres, dweight).

    dweight is accumulated into.  Its dx formula is the true gradient only for
    weight == 1; rmsnorm_bwd is the true gradient for any weight.
    """
    _dev(dy, h, weight, rstd)
    M, N = _rows(dy)
    dx = torch.empty_like(dy)
    dres = torch.empty_like(dy) if want_dres else None
    if dweight is None:
        dweight = torch.zeros_like(weight)
    ws = _norm_ws(M, N, dy.device)
    call("teeny_fused_add_rmsnorm_bwd", _p(dy), _p(h), _p(dx), _p(dres), _p(dweight), _p(weight),
         _p(rstd), M, N, _code(dy), _p(ws), ws.numel(), _stream())
    return dx, dres, dweight


def rmsnorm_bwd(dy, x, weight, rstd, dweight=None):
    """True RMSNorm gradient -> (dx, dweight); dweight is accumulated into."""
    _dev(dy, x, weight, rstd)
    M, N = _rows(dy)
    dx = torch.empty_like(dy)
    if dweight is None:
        dweight = torch.zeros_like(weight)
    ws = _norm_ws(M, N, dy.device)
    call("teeny_rmsnorm_bwd", _p(dy), _p(x), _p(dx), _p(dweight), _p(weight), _p(rstd), M, N,
         _code(dy), _p(ws), ws.numel(), _stream())
    return dx, dweight


# ---------------------------------------------------------------------------
# SwiGLU, embedding
# ---------------------------------------------------------------------------

def swiglu(z: torch.Tensor) -> torch.Tensor:
    """z [..., 2F] (gate || up) -> silu(gate) * up [..., F]."""
    _dev(z)
    M, F2 = _rows(z)
    out = torch.empty(z.shape[:-1] + (F2 // 2,), dtype=z.dtype, device=z.device)
    call("teeny_swiglu_fwd", _p(z), _p(out), M, F2 // 2, _code(z), _stream())
    return out


def swiglu_bwd(grad: torch.Tensor, z: torch.Tensor) -> torch.Tensor:
    _dev(grad, z)
    M, F2 = _rows(z)
    dz = torch.empty_like(z)
    call("teeny_swiglu_bwd", _p(grad), _p(z), _p(dz), M, F2 // 2, _code(z), _stream())
    return dz


def add(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """a + b (the residual add, src/layers/mod.rs:36-48)."""
    _dev(a, b)
    if a.shape != b.shape or a.dtype != b.dtype or not (a.is_contiguous() and b.is_contiguous()):
        raise ValueError("add: a and b must be contiguous tensors of one shape and dtype")
    out = torch.empty_like(a) if out is None else out
    call("teeny_add", _p(a), _p(b), _p(out), a.numel(), _code(a), _stream())
    return out


class SwigluFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, z):
        ctx.save_for_backward(z)
        return swiglu(z)

    @staticmethod
    def backward(ctx, g):
        (z,) = ctx.saved_tensors
        return swiglu_bwd(g.contiguous(), z)


def token_embed(ids: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """ids [...] (int32 or the reference's f32 encoding) -> weight rows [..., d_model]."""
    _dev(ids, weight)
    if ids.dtype == torch.int32:
        idc = TEENY_I32
    elif ids.dtype == torch.float32:
        idc = TEENY_F32
    else:
        raise TypeError("ids must be int32 or float32")
    V, Dm = weight.shape
    out = torch.empty(ids.shape + (Dm,), dtype=weight.dtype, device=weight.device)
    call("teeny_token_embed_fwd", _p(ids), _p(weight), _p(out), ids.numel(), Dm, V, idc,
         _code(weight), _stream())
    return out


# ---------------------------------------------------------------------------
# Llama attention plumbing
# ---------------------------------------------------------------------------

def _ln(rope_base: float) -> float:
    return float(torch.tensor(rope_base, dtype=torch.float32).log().item())


def qkv_rope_split(qkv, q_out, k_cache, v_cache, pos0, n_heads_q: int, n_heads_kv: int,
                   rope_base: float):
    """qkv [B, S, (Hq+2Hkv)*D] -> q_out [B, Hq, S, D] (RoPE) and K (RoPE) / V
    written to caches [B, Hkv, L, D] at rows pos0 .. pos0+S-1.  pos0: an int,
    or a one-element int32 device tensor read when the kernel runs (for
    captured graphs).  q_out None (a dense qkv only): the caches only."""
    if isinstance(qkv, Partials):
        _dev(qkv.slabs, q_out, k_cache, v_cache)
        B, S, _ = qkv.shape
        D = q_out.shape[-1]
        if not isinstance(pos0, torch.Tensor):
            pos0 = torch.tensor([pos0], dtype=torch.int32, device=q_out.device)
        elif pos0.dtype != torch.int32 or not pos0.is_cuda:
            raise TypeError("a device position must be an int32 CUDA tensor")
        call("teeny_qkv_rope_split_partials_dev", _p(qkv.slabs), qkv.n, _p(q_out), _p(k_cache),
             _p(v_cache), B, S, _p(pos0), k_cache.shape[2], n_heads_q, n_heads_kv, D,
             _ln(rope_base), _code(q_out), _stream())
        return
    _dev(qkv, q_out, k_cache, v_cache)
    B, S, _ = qkv.shape
    D = k_cache.shape[-1]
    if isinstance(pos0, torch.Tensor):
        if pos0.dtype != torch.int32 or not pos0.is_cuda:
            raise TypeError("a device position must be an int32 CUDA tensor")
        call("teeny_qkv_rope_split_dev", _p(qkv), _p(q_out), _p(k_cache), _p(v_cache), B, S,
             _p(pos0), k_cache.shape[2], n_heads_q, n_heads_kv, D, _ln(rope_base), _code(qkv),
             _stream())
        return
    call("teeny_qkv_rope_split", _p(qkv), _p(q_out), _p(k_cache), _p(v_cache), B, S, pos0,
         k_cache.shape[2], n_heads_q, n_heads_kv, D, _ln(rope_base), _code(qkv), _stream())


def decode_attention(q, k_cache, v_cache, n_keys: int, softmax_scale: float | None = None,
                     out=None, workspace=None, n_past=None):
    """q [B, Hq, D] (one new row per head) over cache rows 0 .. n_keys-1; with
    n_past (a one-element int32 device tensor, read when the kernel runs) over
    rows 0 .. min(n_past + 1, n_keys) - 1."""
    _dev(q, k_cache, v_cache)
    B, Hq, D = q.shape
    Hkv, L = k_cache.shape[1], k_cache.shape[2]
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    need = _lib.lib().teeny_decode_attention_workspace_bytes(B, Hq, n_keys, D)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    out = torch.empty_like(q) if out is None else out
    if n_past is not None:
        if n_past.dtype != torch.int32 or not n_past.is_cuda:
            raise TypeError("n_past must be an int32 CUDA tensor")
        call("teeny_decode_attention_dev", _p(q), _p(k_cache), _p(v_cache), _p(out), B, Hq, Hkv,
             _p(n_past), n_keys, L, D, scale, _code(q), _p(workspace), workspace.numel(),
             _stream())
        return out
    call("teeny_decode_attention", _p(q), _p(k_cache), _p(v_cache), _p(out), B, Hq, Hkv,
         n_keys, L, D, scale, _code(q), _p(workspace), workspace.numel(), _stream())
    return out


def decode_qkv_attention(qkv: "Partials", k_cache, v_cache, n_past, n_heads_q: int,
                         n_heads_kv: int, rope_base: float, softmax_scale: float | None = None,
                         out=None):
    """A one-token step's attention in one launch: qkv (the QKV projection's
    K-split Partials, [B, 1, (Hq+2Hkv) D]) is split with RoPE at position
    *n_past (a one-element int32 device tensor), k / v are written to cache
    row *n_past, and q attends to rows 0 .. *n_past.  Returns o [B, Hq, D]."""
    if not isinstance(qkv, Partials):
        raise TypeError("decode_qkv_attention takes the QKV projection's K-split slabs")
    _dev(qkv.slabs, k_cache, v_cache)
    if n_past.dtype != torch.int32 or not n_past.is_cuda:
        raise TypeError("n_past must be an int32 CUDA tensor")
    B, S, _ = qkv.shape
    if S != 1:
        raise ValueError("decode_qkv_attention is for one-token steps")
    D, L = k_cache.shape[3], k_cache.shape[2]
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    out = torch.empty((B, n_heads_q, D), dtype=k_cache.dtype, device=k_cache.device) \
        if out is None else out
    call("teeny_decode_qkv_attention_dev", _p(qkv.slabs), qkv.n, _p(k_cache), _p(v_cache),
         _p(out), B, n_heads_q, n_heads_kv, D, L, _p(n_past), _ln(rope_base), scale,
         _code(k_cache), _stream())
    return out


def argmax_rows(x, out=None):
    """x [rows, cols] -> int64 [rows]: the last index of each row's maximum,
    the reference's greedy choice (examples/llama_generate.rs:252-257,
    Iterator::max_by); NaN counts as the maximum."""
    _dev(x)
    x2 = x.reshape(-1, x.shape[-1])
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    rows, cols = x2.shape
    out = torch.empty(rows, dtype=torch.int64, device=x.device) if out is None else out
    call("teeny_argmax_rows", _p(x2), _p(out), rows, cols, _code(x2), _stream())
    return out


def _no_grad(x2: torch.Tensor, w: torch.Tensor) -> bool:
    # the library's linear kernels have no backward: autograd uses torch's GEMM
    return not (torch.is_grad_enabled() and (x2.requires_grad or w.requires_grad))


def _skinny(x2: torch.Tensor, w: torch.Tensor, n_out: int, row_tile: int = 128) -> bool:
    """Shapes the decode-step linear kernels take."""
    M, K = x2.shape
    return (_no_grad(x2, w) and x2.dtype == torch.bfloat16 and w.dtype == torch.bfloat16
            and x2.is_cuda and 1 <= M <= 16 and K % 128 == 0 and n_out % row_tile == 0
            and w.is_contiguous())


def _gemm(x2: torch.Tensor, w: torch.Tensor) -> bool:
    """Shapes teeny_linear_bf16 takes (any M; N and K multiples of 64)."""
    N, K = w.shape
    return (_no_grad(x2, w) and x2.dtype == torch.bfloat16 and w.dtype == torch.bfloat16
            and x2.is_cuda and N % 64 == 0 and K % 64 == 0 and w.is_contiguous())


def _gemm_f32(x2: torch.Tensor, w: torch.Tensor) -> bool:
    """Shapes teeny_linear_f32 takes (any M and N; K a multiple of 4)."""
    return (_no_grad(x2, w) and x2.dtype == torch.float32 and w.dtype == torch.float32
            and x2.is_cuda and w.shape[1] % 4 == 0 and w.is_contiguous())


_own_gemm = threading.local()


@contextlib.contextmanager
def own_gemm():
    """Within this block, products run this library's GEMMs instead of
    hipBLASLt: bf16 products of more than 16 rows teeny_gemm_bf16, fp32
    products teeny_gemm_f32.  That is the rule a captured graph follows by
    itself (the linear entry points never run hipBLASLt under capture),
    applied to eager calls so that an eager step and its graph replay run
    the same kernels."""
    prev = getattr(_own_gemm, "on", False)
    _own_gemm.on = True
    try:
        yield
    finally:
        _own_gemm.on = prev


class StreamWeight:
    """A bf16 weight W [N, K] with its streaming-layout copy
    (teeny_linear_stream_layout_bf16: the order in which the decode-step
    kernels load it, one contiguous KiB per load instruction).  linear,
    linear_swiglu and linear_split take it in place of the tensor: products
    of up to 16 rows read the copy (teeny_linear_*sl_bf16, the same outputs),
    other products the row-major W.  Costs one more copy of W.  The copy is
    made once, here: after an in-place change of W, make a new StreamWeight."""

    def __init__(self, w: torch.Tensor):
        if w.dim() != 2 or w.dtype != torch.bfloat16 or not w.is_cuda or not w.is_contiguous():
            raise ValueError("StreamWeight: a contiguous bf16 [N, K] device tensor")
        N, K = w.shape
        if N % 16 or K % 128:
            raise ValueError("StreamWeight: N must be a multiple of 16 and K of 128")
        self.w = w
        self.s = torch.empty_like(w)
        call("teeny_linear_stream_layout_bf16", _p(w), _p(self.s), N, K, _stream())

    @property
    def shape(self):
        return self.w.shape


def _row_major(w):
    return w.w if isinstance(w, StreamWeight) else w


def linear(x: torch.Tensor, w) -> torch.Tensor:
    """y = x w^T (src/layers/mod.rs:54-58; w [out, in]) through the library:
    bf16 by teeny_linear_bf16 (up to 16 rows stream the weight through the
    decode kernels, more rows run hipBLASLt, or this library's GEMM under
    own_gemm()), fp32 (the reference's precision) by teeny_linear_f32.
    Products that need a gradient use torch's GEMM (the library's linear
    kernels have no backward).  w may be a StreamWeight."""
    x2 = x.reshape(-1, x.shape[-1])
    N, K = w.shape
    if K != x2.shape[1]:
        raise ValueError(f"linear: x has {x2.shape[1]} features, w expects {K}")
    if isinstance(w, StreamWeight):
        if _skinny(x2, w.w, N):
            x2 = x2.contiguous()
            y = torch.empty((x2.shape[0], N), dtype=x.dtype, device=x.device)
            call("teeny_linear_sl_bf16", _p(x2), _p(w.s), _p(y), x2.shape[0], N, K, _stream())
            return y.view(*x.shape[:-1], N)
        w = w.w
    if _gemm_f32(x2, w):
        x2 = x2.contiguous()
        y = torch.empty((x2.shape[0], N), dtype=x.dtype, device=x.device)
        fn = "teeny_gemm_f32" if getattr(_own_gemm, "on", False) else "teeny_linear_f32"
        call(fn, _p(x2), _p(w), _p(y), x2.shape[0], N, K, _stream())
        return y.view(*x.shape[:-1], N)
    if not _gemm(x2, w):
        return torch.nn.functional.linear(x, w)
    x2 = x2.contiguous()
    y = torch.empty((x2.shape[0], N), dtype=x.dtype, device=x.device)
    fn = ("teeny_gemm_bf16" if x2.shape[0] > 16 and getattr(_own_gemm, "on", False)
          else "teeny_linear_bf16")
    call(fn, _p(x2), _p(w), _p(y), x2.shape[0], N, K, _stream())
    return y.view(*x.shape[:-1], N)


def gemm_f32(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """x w^T in fp32 through this library's own GEMM (teeny_gemm_f32)."""
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    N, K = w.shape
    if K != x2.shape[1] or not _gemm_f32(x2, w):
        raise ValueError("gemm_f32: fp32 x [.., K] and contiguous w [N, K], K a multiple of 4")
    y = torch.empty((x2.shape[0], N), dtype=x.dtype, device=x.device)
    call("teeny_gemm_f32", _p(x2), _p(w), _p(y), x2.shape[0], N, K, _stream())
    return y.view(*x.shape[:-1], N)


def gemm_own(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """x w^T through this library's own matrix-core GEMM (teeny_gemm_bf16),
    any row count, bf16, no gradients (teeny_linear_bf16 hands prompt sizes
    to hipBLASLt instead)."""
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    N, K = w.shape
    if K != x2.shape[1] or not _gemm(x2, w):
        raise ValueError("gemm_own: bf16 x [.., K] and contiguous w [N, K], N and K multiples of 64")
    y = torch.empty((x2.shape[0], N), dtype=x.dtype, device=x.device)
    call("teeny_gemm_bf16", _p(x2), _p(w), _p(y), x2.shape[0], N, K, _stream())
    return y.view(*x.shape[:-1], N)


def linear_swiglu(x: torch.Tensor, w_gate_up) -> torch.Tensor:
    """swiglu(x w_gate_up^T) (src/layers/ffn.rs:47-56).  Up to 16 bf16 rows
    without gradients: one launch of teeny_linear_swiglu_bf16 (the decode
    kernel with the SwiGLU fused).  More rows: the linear entry point
    (hipBLASLt) and then the SwiGLU kernel, measured faster than the own GEMM
    with the SwiGLU epilogue (1.40 against 1.52 ms at 8192 x 28672 x 4096);
    other cases: the GEMM followed by the SwiGLU kernel.  w_gate_up may be a
    StreamWeight."""
    x2 = x.reshape(-1, x.shape[-1])
    N2, K = w_gate_up.shape
    if K != x2.shape[1] or N2 % 2:
        raise ValueError("linear_swiglu: weight must be [2F, in] with in = x's features")
    F = N2 // 2
    w = _row_major(w_gate_up)
    if not _gemm(x2, w) or not _skinny(x2, w, F, row_tile=64):
        return swiglu(linear(x, w))
    x2 = x2.contiguous()
    y = torch.empty((x2.shape[0], F), dtype=x.dtype, device=x.device)
    if isinstance(w_gate_up, StreamWeight):
        call("teeny_linear_swiglu_sl_bf16", _p(x2), _p(w_gate_up.s), _p(y), x2.shape[0], F, K,
             _stream())
    else:
        call("teeny_linear_swiglu_bf16", _p(x2), _p(w), _p(y), x2.shape[0], F, K, _stream())
    return y.view(*x.shape[:-1], F)


class Partials:
    """A linear layer's output left as fp32 slabs [n, M, N] of a K split; the
    consumer (fused_add_rmsnorm, qkv_rope_split) sums them in slab order and
    rounds to `dtype`, the product's storage type."""

    def __init__(self, slabs: torch.Tensor, shape, dtype):
        self.slabs, self.shape, self.dtype = slabs, tuple(shape), dtype

    @property
    def n(self) -> int:
        return self.slabs.shape[0]

    def sum(self) -> torch.Tensor:
        """The product itself (for checks; consumers read the slabs)."""
        return self.slabs.sum(0, dtype=torch.float32).to(self.dtype).view(self.shape)


def _k_split(K: int, N: int) -> int:
    """K per slab, in whole 128-wide steps.  The 128-feature workgroups times
    the slabs are spread over 256 CUs; the slab count (at most 16) minimises
    the busiest CU's work, ceil(workgroups / 256) * (steps per slab + 2), the
    2 standing for a workgroup's fixed cost, and ties go to fewer slabs (each
    slab costs the consumer a read)."""
    rows, steps = N // 128, K // 128
    best = min(range(1, 17), key=lambda n: (-(-rows * n // 256) * (-(-steps // n) + 2), n))
    return -(-steps // best) * 128


def linear_split(x: torch.Tensor, w, k_split: int | None = None):
    """x w^T as Partials where the decode kernels take the shape (up to 16
    bf16 rows), else the GEMM's tensor.  k_split (a multiple of 128) sets K
    per slab; by default it is chosen to spread the work over the CUs.  w may
    be a StreamWeight."""
    x2 = x.reshape(-1, x.shape[-1])
    N, K = w.shape
    if K != x2.shape[1]:
        raise ValueError(f"linear: x has {x2.shape[1]} features, w expects {K}")
    if not _skinny(x2, _row_major(w), N):
        return linear(x, _row_major(w))
    x2 = x2.contiguous()
    ks = _k_split(K, N) if k_split is None else k_split
    n = _lib.lib().teeny_linear_partials_count(K, ks)
    slabs = torch.empty((n, x2.shape[0], N), dtype=torch.float32, device=x.device)
    if isinstance(w, StreamWeight):
        call("teeny_linear_partials_sl_bf16", _p(x2), _p(w.s), _p(slabs), x2.shape[0], N, K, ks,
             _stream())
    else:
        call("teeny_linear_partials_bf16", _p(x2), _p(w), _p(slabs), x2.shape[0], N, K, ks,
             _stream())
    return Partials(slabs, (*x.shape[:-1], N), x.dtype)

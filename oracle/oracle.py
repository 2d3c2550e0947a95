"""ctypes binding of the C oracle (oracle.c) plus small numpy helpers.

TEST INFRASTRUCTURE ONLY: the parity reference for the HIP library and the
timed CPU baseline.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only to check results.

All arrays are numpy, C-contiguous.  Attention tensors use the reference's
[BH, N_CTX, HEAD_DIM] layout (src/kernels/flash_attn2.rs:23), written here as
[B, H, S, D] with the batch split out.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lib = None

_F = ctypes.POINTER(ctypes.c_float)
_D = ctypes.POINTER(ctypes.c_double)
_V = ctypes.c_void_p
_I = ctypes.c_int


def build() -> None:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.orc_fa2_fwd.argtypes = [_F, _F, _F, _F, _F] + [_I] * 6 + [ctypes.c_float, _I, _I, _I]
        L.orc_fa2_bwd.argtypes = [_F] * 9 + [_I] * 6 + [ctypes.c_float, _I, _I, _I]
        L.orc_attn_dense_f64.argtypes = [_F, _F, _F, _F, _D, _D, _D, _D, _D] + [_I] * 6 + [ctypes.c_double, _I]
        L.orc_rope_inv_freq.argtypes = [_I, _I, ctypes.c_float]
        L.orc_rope_inv_freq.restype = ctypes.c_float
        L.orc_rope.argtypes = [_F, _F, _I, _I, _I, ctypes.c_float, _I]
        L.orc_rope_at.argtypes = [_F, _F, _I, _I, _I, ctypes.c_float, _I, _I]
        L.orc_transpose_heads.argtypes = [_V, _V, _I, _I, _I, _I, _I, _I]
        L.orc_fused_add_rmsnorm_fwd.argtypes = [_F] * 6 + [_I, _I, ctypes.c_float]
        L.orc_rmsnorm_fwd.argtypes = [_F] * 4 + [_I, _I, ctypes.c_float]
        L.orc_fused_add_rmsnorm_bwd.argtypes = [_F] * 7 + [_I, _I]
        L.orc_rmsnorm_bwd.argtypes = [_F] * 6 + [_I, _I]
        L.orc_swiglu_fwd.argtypes = [_F, _F, _I, _I]
        L.orc_swiglu_bwd.argtypes = [_F, _F, _F, _I, _I]
        L.orc_token_embed.argtypes = [_F, _F, _F, _I, _I]
        L.orc_num_threads.restype = _I
        L.orc_set_num_threads.argtypes = [_I]
        _lib = L
    return _lib


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(_F)


def _pf(a):
    return a.ctypes.data_as(_F) if a is not None else ctypes.cast(None, _F)


def num_threads() -> int:
    return lib().orc_num_threads()


def set_num_threads(n: int) -> None:
    lib().orc_set_num_threads(int(n))


# --------------------------------------------------------------------------
# bf16 helpers
# --------------------------------------------------------------------------

def bf16_round(x) -> np.ndarray:
    """Round fp32 values to the nearest bf16 (ties to even); returns fp32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


# --------------------------------------------------------------------------
# Flash attention
# --------------------------------------------------------------------------

def fa2_fwd(q, k, v, scale: float, causal: bool, all_keys: bool = False, q_offset: int = 0):
    """q [B,Hq,Nq,D], k/v [B,Hkv,Nk,D] -> (o [B,Hq,Nq,D], lse [B,Hq,Nq]) fp32.

    q_offset: causal position of q row 0 (to check a slice of query rows)."""
    q, pq = _f32(q)
    k, pk = _f32(k)
    v, pv = _f32(v)
    B, Hq, Nq, D = q.shape
    Hkv, Nk = k.shape[1], k.shape[2]
    o = np.empty_like(q)
    lse = np.empty((B, Hq, Nq), np.float32)
    lib().orc_fa2_fwd(pq, pk, pv, _pf(o), _pf(lse), B, Hq, Hkv, Nq, Nk, D,
                      float(scale), int(causal), int(all_keys), int(q_offset))
    return o, lse


def fa2_bwd(q, k, v, o, do, lse, scale: float, causal: bool, all_keys: bool = False,
            q_offset: int = 0):
    """Reference backward -> (dq, dk, dv) fp32."""
    q, pq = _f32(q)
    k, pk = _f32(k)
    v, pv = _f32(v)
    o, po = _f32(o)
    do, pdo = _f32(do)
    lse, pl = _f32(lse)
    B, Hq, Nq, D = q.shape
    Hkv, Nk = k.shape[1], k.shape[2]
    dq = np.empty_like(q)
    dk = np.empty_like(k)
    dv = np.empty_like(v)
    lib().orc_fa2_bwd(pq, pk, pv, po, pdo, pl, _pf(dq), _pf(dk), _pf(dv),
                      B, Hq, Hkv, Nq, Nk, D, float(scale), int(causal), int(all_keys),
                      int(q_offset))
    return dq, dk, dv


def attn_dense_f64(q, k, v, scale: float, causal: bool, do=None):
    """Textbook attention in float64 -> dict(o, lse[, dq, dk, dv])."""
    q, pq = _f32(q)
    k, pk = _f32(k)
    v, pv = _f32(v)
    B, Hq, Nq, D = q.shape
    Hkv, Nk = k.shape[1], k.shape[2]
    o = np.empty(q.shape, np.float64)
    lse = np.empty((B, Hq, Nq), np.float64)
    out = {"o": o, "lse": lse}
    dp = ctypes.cast(None, _F)
    dq = dk = dv = None
    if do is not None:
        do, dp = _f32(do)
        dq = np.empty(q.shape, np.float64)
        dk = np.empty(k.shape, np.float64)
        dv = np.empty(v.shape, np.float64)
        out.update(dq=dq, dk=dk, dv=dv)

    def pdd(a):
        return a.ctypes.data_as(_D) if a is not None else ctypes.cast(None, _D)

    lib().orc_attn_dense_f64(pq, pk, pv, dp, pdd(o), pdd(lse), pdd(dq), pdd(dk), pdd(dv),
                             B, Hq, Hkv, Nq, Nk, D, float(scale), int(causal))
    return out


# --------------------------------------------------------------------------
# RoPE / transpose
# --------------------------------------------------------------------------

def rope_inv_freq(d: int, ln_base: float) -> np.ndarray:
    return np.array([lib().orc_rope_inv_freq(k, d, ln_base) for k in range(d // 2)], np.float32)


def rope(x, ln_base: float, backward: bool = False, pos0: int = 0) -> np.ndarray:
    """x [..., S, D] (leading dims flattened to BH) -> rotated copy (fp32);
    row s of each slice at position pos0 + s."""
    x, px = _f32(x)
    S, D = x.shape[-2], x.shape[-1]
    bh = int(np.prod(x.shape[:-2])) if x.ndim > 2 else 1
    y = np.empty_like(x)
    if pos0:
        lib().orc_rope_at(px, _pf(y), bh, S, D, float(ln_base), int(backward), int(pos0))
    else:
        lib().orc_rope(px, _pf(y), bh, S, D, float(ln_base), int(backward))
    return y


def transpose_heads(src: np.ndarray, batch: int, seq: int, heads: int, head_dim: int,
                    merge: bool = False) -> np.ndarray:
    """Byte-exact [B,S,H,D] -> [B,H,S,D] (or the reverse with merge=True)."""
    src = np.ascontiguousarray(src)
    dst = np.empty_like(src)
    lib().orc_transpose_heads(src.ctypes.data, dst.ctypes.data, batch, seq, heads, head_dim,
                              src.itemsize, int(merge))
    if merge:
        return dst.reshape(batch, seq, heads * head_dim)
    return dst.reshape(batch, heads, seq, head_dim)


# --------------------------------------------------------------------------
# Norms, SwiGLU, embedding
# --------------------------------------------------------------------------

def fused_add_rmsnorm_fwd(x, res, w, eps: float):
    x, px = _f32(x)
    res, pr = _f32(res)
    w, pw = _f32(w)
    M, N = x.shape
    y = np.empty_like(x)
    h = np.empty_like(x)
    rstd = np.empty(M, np.float32)
    lib().orc_fused_add_rmsnorm_fwd(px, pr, _pf(y), _pf(h), _pf(rstd), pw, M, N, float(eps))
    return y, h, rstd


def rmsnorm_fwd(x, w, eps: float):
    x, px = _f32(x)
    w, pw = _f32(w)
    M, N = x.shape
    y = np.empty_like(x)
    rstd = np.empty(M, np.float32)
    lib().orc_rmsnorm_fwd(px, _pf(y), _pf(rstd), pw, M, N, float(eps))
    return y, rstd


def fused_add_rmsnorm_bwd(dy, h, w, rstd, dw_in=None):
    dy, pdy = _f32(dy)
    h, ph = _f32(h)
    w, pw = _f32(w)
    rstd, prs = _f32(rstd)
    M, N = dy.shape
    dx = np.empty_like(dy)
    dres = np.empty_like(dy)
    dw = np.zeros(N, np.float32) if dw_in is None else np.array(dw_in, np.float32, copy=True)
    lib().orc_fused_add_rmsnorm_bwd(pdy, ph, _pf(dx), _pf(dres), _pf(dw), pw, prs, M, N)
    return dx, dres, dw


def rmsnorm_bwd(dy, h, w, rstd, dw_in=None):
    """True RMSNorm gradient -> (dx, dw); dw accumulates onto dw_in."""
    dy, pdy = _f32(dy)
    h, ph = _f32(h)
    w, pw = _f32(w)
    rstd, prs = _f32(rstd)
    M, N = dy.shape
    dx = np.empty_like(dy)
    dw = np.zeros(N, np.float32) if dw_in is None else np.array(dw_in, np.float32, copy=True)
    lib().orc_rmsnorm_bwd(pdy, ph, _pf(dx), _pf(dw), pw, prs, M, N)
    return dx, dw


def swiglu_fwd(z):
    z, pz = _f32(z)
    M, F2 = z.shape
    out = np.empty((M, F2 // 2), np.float32)
    lib().orc_swiglu_fwd(pz, _pf(out), M, F2 // 2)
    return out


def swiglu_bwd(grad, z):
    grad, pg = _f32(grad)
    z, pz = _f32(z)
    M, F2 = z.shape
    dz = np.empty_like(z)
    lib().orc_swiglu_bwd(pg, pz, _pf(dz), M, F2 // 2)
    return dz


def token_embed(ids, w):
    ids, pi = _f32(ids)
    w, pw = _f32(w)
    S = ids.shape[0]
    out = np.empty((S, w.shape[1]), np.float32)
    lib().orc_token_embed(pi, pw, _pf(out), S, w.shape[1])
    return out


# --------------------------------------------------------------------------
# Golden fixtures (raw little-endian f32, as the reference's tests read them:
# tests/kernel_execution.rs:39-47)
# --------------------------------------------------------------------------

GOLDEN = os.path.join(os.path.dirname(HERE), "tests", "golden")


def load_fixture(rel: str) -> np.ndarray:
    return np.fromfile(os.path.join(GOLDEN, rel), dtype="<f4")

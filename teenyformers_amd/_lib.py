"""ctypes binding of libteeny_hip.so (the C ABI declared in include/teeny_hip.h).

There is no fallback: if the library is not built, or a call returns an
error code, a TeenyError is raised.
"""
from __future__ import annotations

import ctypes
import os
import re

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libteeny_hip.so")
HEADER = os.path.join(os.path.dirname(PKG), "include", "teeny_hip.h")

TEENY_F32, TEENY_BF16, TEENY_I32 = 0, 1, 2
TEENY_GRAD_F32 = 0x100  # or-ed into a bf16 backward's dtype: fp32 dq/dk/dv


class TeenyError(RuntimeError):
    def __init__(self, what: str, code: int, hip_error: int = 0):
        self.code = code
        self.hip_error = hip_error
        msg = f"{what} failed: {strerror(code)} (code {code})"
        if hip_error:
            msg += f", hip error {hip_error}"
        super().__init__(msg)


_lib = None

_p = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t

_SIGNATURES = {
    "teeny_abi_version": ([], _i),
    "teeny_strerror": ([_i], ctypes.c_char_p),
    "teeny_last_hip_error": ([], _i),
    "teeny_init": ([], _i),
    "teeny_profile_enable": ([_i], _i),
    "teeny_profile_kernel_stats": ([ctypes.c_char_p, ctypes.POINTER(_i),
                                    ctypes.POINTER(ctypes.c_double)], _i),
    "teeny_profile_kernel_names": ([ctypes.c_char_p, _sz], _i),
    "teeny_causal_flash_attn2_fwd": ([_p] * 5 + [_i, _i, _f, _f, _i, _i, _i, _i, _i, _p], _i),
    "teeny_flash_attn2_fwd": ([_p] * 5 + [_i, _i, _f, _f, _i, _i, _i, _i, _i, _p], _i),
    "teeny_flash_attn2_fwd_merged": ([_p] * 5 + [_i, _i, _f, _f, _i, _i, _i, _i, _i, _i, _p], _i),
    "teeny_flash_attn2_fwd_qkv": ([_p] * 6 + [_i, _i, _f, _f, _i, _i, _i, _i, _i, _i, _p], _i),
    "teeny_rope_table": ([_p, _i, _i, _f, _p], _i),
    "teeny_causal_flash_attn2_bwd": ([_p] * 9 + [_i, _i, _f, _i, _i, _i, _i, _i, _p, _sz, _p], _i),
    "teeny_flash_attn2_bwd": ([_p] * 9 + [_i, _i, _f, _i, _i, _i, _i, _i, _p, _sz, _p], _i),
    "teeny_flash_attn2_bwd_workspace_bytes": ([_i, _i, _i, _i, _i], _sz),
    "teeny_scratch_bytes": ([], _sz),
    "teeny_causal_flash_attn2_bwd_noalloc": ([_p] * 9 + [_i, _i, _f, _i, _i, _i, _i, _i, _p], _i),
    "teeny_flash_attn2_bwd_workspace_bytes_gqa": ([_i] * 7, _sz),
    "teeny_rope_fwd": ([_p, _p, _i, _f, _i, _i, _i, _p], _i),
    "teeny_rope_bwd": ([_p, _p, _i, _f, _i, _i, _i, _p], _i),
    "teeny_transpose_heads": ([_p, _p, _i, _i, _i, _i, _i, _p], _i),
    "teeny_merge_heads": ([_p, _p, _i, _i, _i, _i, _i, _p], _i),
    "teeny_fused_add_rmsnorm_fwd": ([_p] * 6 + [_i, _i, _f, _i, _p], _i),
    "teeny_fused_add_rmsnorm_bwd": ([_p] * 7 + [_i, _i, _i, _p, _sz, _p], _i),
    "teeny_fused_add_rmsnorm_bwd_workspace_bytes": ([_i, _i], _sz),
    "teeny_rmsnorm_fwd": ([_p] * 4 + [_i, _i, _f, _i, _p], _i),
    "teeny_rmsnorm_bwd": ([_p] * 6 + [_i, _i, _i, _p, _sz, _p], _i),
    "teeny_swiglu_fwd": ([_p, _p, _i, _i, _i, _p], _i),
    "teeny_swiglu_bwd": ([_p, _p, _p, _i, _i, _i, _p], _i),
    "teeny_add": ([_p, _p, _p, ctypes.c_long, _i, _p], _i),
    "teeny_token_embed_fwd": ([_p, _p, _p, _i, _i, _i, _i, _i, _p], _i),
    "teeny_qkv_rope_split": ([_p] * 4 + [_i] * 7 + [_f, _i, _p], _i),
    "teeny_decode_attention_workspace_bytes": ([_i] * 4, _sz),
    "teeny_decode_attention": ([_p] * 4 + [_i] * 6 + [_f, _i, _p, _sz, _p], _i),
    "teeny_qkv_rope_split_dev": ([_p] * 4 + [_i, _i, _p] + [_i] * 4 + [_f, _i, _p], _i),
    "teeny_decode_attention_dev": ([_p] * 4 + [_i] * 3 + [_p] + [_i] * 3
                                   + [_f, _i, _p, _sz, _p], _i),
    "teeny_decode_qkv_attention_dev": ([_p, _i, _p, _p, _p] + [_i] * 5 + [_p, _f, _f, _i, _p],
                                       _i),
    "teeny_argmax_rows": ([_p, _p, _i, _i, _i, _p], _i),
    "teeny_linear_bf16": ([_p, _p, _p, _i, _i, _i, _p], _i),
    "teeny_gemm_bf16": ([_p, _p, _p, _i, _i, _i, _p], _i),
    "teeny_linear_swiglu_bf16": ([_p, _p, _p, _i, _i, _i, _p], _i),
    "teeny_linear_f32": ([_p, _p, _p, _i, _i, _i, _p], _i),
    "teeny_gemm_f32": ([_p, _p, _p, _i, _i, _i, _p], _i),
    "teeny_linear_partials_count": ([_i, _i], _i),
    "teeny_linear_partials_bf16": ([_p, _p, _p, _i, _i, _i, _i, _p], _i),
    "teeny_linear_stream_layout_bf16": ([_p, _p, _i, _i, _p], _i),
    "teeny_linear_sl_bf16": ([_p, _p, _p, _i, _i, _i, _p], _i),
    "teeny_linear_swiglu_sl_bf16": ([_p, _p, _p, _i, _i, _i, _p], _i),
    "teeny_linear_partials_sl_bf16": ([_p, _p, _p, _i, _i, _i, _i, _p], _i),
    "teeny_fused_add_rmsnorm_partials_fwd": ([_p, _i, _p, _p, _p, _p, _p, _i, _i, _f, _i, _p], _i),
    "teeny_qkv_rope_split_partials_dev": ([_p, _i, _p, _p, _p, _i, _i, _p, _i, _i, _i, _i, _f,
                                           _i, _p], _i),
}


def lib() -> ctypes.CDLL:
    """Load libteeny_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is not built; run `python -m teenyformers_amd.build` "
                "(there is no CPU fallback for the HIP kernels)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def strerror(code: int) -> str:
    try:
        return lib().teeny_strerror(code).decode()
    except Exception:  # pragma: no cover - only when the library itself is missing
        return "unknown"


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise TeenyError(what, rc, lib().teeny_last_hip_error())


def call(name: str, *args) -> None:
    """Call a status-returning entry point and raise on a nonzero status."""
    check(getattr(lib(), name)(*args), name)


def profile_enable(on: bool) -> None:
    call("teeny_profile_enable", int(bool(on)))


def profile_stats() -> dict[str, tuple[int, float]]:
    """{kernel symbol: (launches, total ms)} for the launches recorded since
    profile_enable(True).  Synchronises on the recorded events."""
    buf = ctypes.create_string_buffer(1 << 16)
    call("teeny_profile_kernel_names", buf, len(buf))
    out = {}
    for name in buf.value.decode().split():
        n, ms = _i(), ctypes.c_double()
        call("teeny_profile_kernel_stats", name.encode(), ctypes.byref(n), ctypes.byref(ms))
        out[name] = (n.value, ms.value)
    return out


def header_functions() -> list[str]:
    """Names of the functions declared in include/teeny_hip.h."""
    with open(HEADER) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(teeny_[a-z0-9_]+)\s*\(", text)))

"""The no-allocation causal FA2 backward (teeny_causal_flash_attn2_bwd_noalloc,
whose workspace is the library's static per-device scratch array) against
the allocating entry point teeny_causal_flash_attn2_bwd given a workspace of
the same size: the same kernels on the same inputs, so the gradients must be
bit-identical.  Two calls in a row, the second on a smaller problem (the
array keeps the first call's contents, which the second must not depend
on), for bf16 and for bf16 with fp32 gradients; the first result is also
held to the oracle's bf16 bar."""
import ctypes
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from teenyformers_amd import _lib, ops

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _inputs(B, Hq, Hkv, S, D, seed):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn((B, Hq, S, D), generator=gen, device="cuda").to(torch.bfloat16)
    k = torch.randn((B, Hkv, S, D), generator=gen, device="cuda").to(torch.bfloat16)
    v = torch.randn((B, Hkv, S, D), generator=gen, device="cuda").to(torch.bfloat16)
    do = torch.randn((B, Hq, S, D), generator=gen, device="cuda").to(torch.bfloat16)
    return q, k, v, do


def _noalloc(q, k, v, o, lse, do, scale, grad_f32):
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    gdt = torch.float32 if grad_f32 else torch.bfloat16
    dq = torch.full(q.shape, float("nan"), dtype=gdt, device="cuda")
    dk = torch.full(k.shape, float("nan"), dtype=gdt, device="cuda")
    dv = torch.full(v.shape, float("nan"), dtype=gdt, device="cuda")
    code = _lib.TEENY_BF16 | (_lib.TEENY_GRAD_F32 if grad_f32 else 0)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = _lib.lib().teeny_causal_flash_attn2_bwd_noalloc(
        _p(q), _p(k), _p(v), _p(o), _p(do), _p(lse), _p(dq), _p(dk), _p(dv), S, S, scale, B, Hq,
        Hkv, D, code, stream)
    assert rc == 0, _lib.strerror(rc)
    return dq, dk, dv


@pytest.mark.parametrize("grad_f32", [False, True])
def test_noalloc_bwd_matches_allocating_entry(cuda, grad_f32):
    L = _lib.lib()
    scratch = L.teeny_scratch_bytes()
    assert scratch == 16 << 20
    # (B, Hq, Hkv, S, D): a GQA problem whose dK/dV head split fits in the
    # array, then a smaller MHA one at the other head dim
    for i, (B, Hq, Hkv, S, D) in enumerate([(2, 8, 2, 1000, 128), (1, 4, 4, 300, 64)]):
        print(f"noalloc call {i}: B{B} Hq{Hq} Hkv{Hkv} S{S} D{D} grad_f32={grad_f32}", flush=True)
        q, k, v, do = _inputs(B, Hq, Hkv, S, D, seed=90 + i)
        scale = 1.0 / math.sqrt(D)
        o, lse = ops.flash_attn2_fwd(q, k, v, scale, True)
        ws = torch.empty(scratch, dtype=torch.uint8, device="cuda")
        want = ops.flash_attn2_bwd(q, k, v, o, lse, do, scale, True, workspace=ws,
                                   grad_f32=grad_f32)
        got = _noalloc(q, k, v, o, lse, do, scale, grad_f32)
        torch.cuda.synchronize()
        for name, g, w in zip(("dQ", "dK", "dV"), got, want):
            assert torch.equal(g, w), name
        if i == 0:  # and the oracle's bf16 bar (the backward's own O and LSE)
            h = lambda t: t.float().cpu().numpy()  # noqa: E731
            dqe, dke, dve = O.fa2_bwd(h(q), h(k), h(v), h(o), h(do), h(lse), scale, True)
            for name, g, w in zip(("dQ", "dK", "dV"), got, (dqe, dke, dve)):
                g = h(g)
                err = float(np.abs(g - w).max())
                rel = float(np.linalg.norm(g - w) / np.linalg.norm(w))
                assert rel <= 5e-3 and err <= 2e-2 * max(1.0, float(np.abs(w).max()) / 4), \
                    f"{name}: max abs {err:.3e} rel-L2 {rel:.3e}"

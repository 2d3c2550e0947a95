"""The no-allocation causal FA2 backward (teeny_causal_flash_attn2_bwd_noalloc,
whose workspace is the library's static per-device scratch array) against
the allocating entry point teeny_causal_flash_attn2_bwd given a workspace of
the same size: the same kernels on the same inputs, so the gradients must be
bit-identical.  Two calls in a row, the second on a smaller problem (the
array keeps the first call's contents, which the second must not depend
on), for bf16 and for bf16 with fp32 gradients; the second result is also
held to the oracle's bf16 bar.  The first problem's dK/dV head split (fp32
partials in the array, then the merge kernel) runs inside the array.  And
the entry point captured in a HIP graph: every replay equals the eager
result, with other calls overwriting the array between replays."""
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
    # array (12288 query rows, the split's lower bound, and a group of 2: 2
    # partial sums of dK and dV, 12 MiB), then a smaller MHA one
    cases = [(1, 2, 1, 12288, 64), (1, 4, 4, 300, 64)]
    B, Hq, Hkv, S, D = cases[0]
    base = L.teeny_flash_attn2_bwd_workspace_bytes(S, B, Hq, D, _lib.TEENY_BF16)
    split = L.teeny_flash_attn2_bwd_workspace_bytes_gqa(S, S, B, Hq, Hkv, D, _lib.TEENY_BF16)
    assert base < split <= scratch, (base, split)
    for i, (B, Hq, Hkv, S, D) in enumerate(cases):
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
        if i == 1:  # and the oracle's bf16 bar (the backward's own O and LSE)
            h = lambda t: t.float().cpu().numpy()  # noqa: E731
            dqe, dke, dve = O.fa2_bwd(h(q), h(k), h(v), h(o), h(do), h(lse), scale, True)
            for name, g, w in zip(("dQ", "dK", "dV"), got, (dqe, dke, dve)):
                g = h(g)
                err = float(np.abs(g - w).max())
                rel = float(np.linalg.norm(g - w) / np.linalg.norm(w))
                assert rel <= 5e-3 and err <= 2e-2 * max(1.0, float(np.abs(w).max()) / 4), \
                    f"{name}: max abs {err:.3e} rel-L2 {rel:.3e}"


def test_noalloc_bwd_under_graph_capture(cuda):
    """The entry point recorded in a HIP graph (it loads and allocates
    nothing, and clears nothing with a memset node): three replays, each
    after eager calls of the same entry point on another problem have
    overwritten the shared array, give the eager gradients bit for bit."""
    B, Hq, Hkv, S, D = 1, 2, 1, 12288, 64  # with the dK/dV head split in the array
    q, k, v, do = _inputs(B, Hq, Hkv, S, D, seed=95)
    scale = 1.0 / math.sqrt(D)
    o, lse = ops.flash_attn2_fwd(q, k, v, scale, True)
    want = _noalloc(q, k, v, o, lse, do, scale, False)
    q2, k2, v2, do2 = _inputs(1, 4, 4, 700, 128, seed=96)
    o2, lse2 = ops.flash_attn2_fwd(q2, k2, v2, 1.0 / math.sqrt(128), True)
    torch.cuda.synchronize()

    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        rc = _lib.lib().teeny_causal_flash_attn2_bwd_noalloc(
            _p(q), _p(k), _p(v), _p(o), _p(do), _p(lse), _p(dq), _p(dk), _p(dv), S, S, scale, B,
            Hq, Hkv, D, _lib.TEENY_BF16, stream)
    assert rc == 0, _lib.strerror(rc)
    for r in range(3):
        # another problem through the same array, eagerly, between replays
        _noalloc(q2, k2, v2, o2, lse2, do2, 1.0 / math.sqrt(128), r % 2 == 1)
        for t in (dq, dk, dv):
            t.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        print(f"noalloc graph replay {r}", flush=True)
        for name, got, w in zip(("dQ", "dK", "dV"), (dq, dk, dv), want):
            assert torch.equal(got, w), f"replay {r}: {name}"

"""GPU parity of the bandwidth kernels (RoPE, head transposes, RMSNorm,
SwiGLU, embedding) against the CPU oracle, through the C ABI.

Bars: bit-exact for transposes and the gather; <= 1e-5 max abs for fp32
math; bf16 outputs within one bf16 rounding of the oracle's fp32 result on
the same bf16-rounded inputs.
"""
import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from teenyformers_amd import ops

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5


def f32_ln(x):
    return float(np.log(np.float32(x)).astype(np.float32))


def randn(seed, *shape):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def dev(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def host(t):
    return t.float().cpu().numpy()


def f32_close(got, want):
    """fp32 bar for row reductions: 1e-5 absolute, or 2e-6 of the output
    scale when outputs exceed 5 (a reduction over N terms may round
    differently from the oracle's sequential sum)."""
    return float(np.abs(got - want).max()) <= max(F32_TOL, 2e-6 * float(np.abs(want).max()))


def bf16_close(got, want):
    """|got - want| <= one bf16 ulp of want (plus a tiny absolute floor)."""
    ulp = np.abs(want) * 2.0 ** -8 + 1e-30
    return np.all(np.abs(got - want) <= ulp + 1e-6)


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------

def test_rope_reference_fixture(cuda):
    meta = json.load(open(os.path.join(O.GOLDEN, "rope", "meta.json")))
    x = O.load_fixture("rope/input.bin").reshape(meta["bh"], meta["s"], meta["head_dim"])
    want = O.load_fixture("rope/output.bin").reshape(x.shape)
    got = host(ops.rope(dev(x), meta["rope_base"]))
    assert np.abs(got - want).max() < 1e-4  # the reference's own tolerance
    assert np.abs(got - want).max() < 1e-6


@pytest.mark.parametrize("bh,s,d,base", [(4, 128, 64, 1e4), (6, 333, 128, 5e5),
                                         (2, 16384, 128, 5e5), (3, 50, 16, 1e4)])
def test_rope_f32(cuda, bh, s, d, base):
    x = randn(1, bh, s, d)
    want = O.rope(x, f32_ln(base))
    got = host(ops.rope(dev(x), base))
    assert np.abs(got - want).max() <= F32_TOL
    back = host(ops.rope(dev(got), base, backward=True))
    assert np.abs(back - O.rope(got, f32_ln(base), backward=True)).max() <= F32_TOL


@pytest.mark.parametrize("bh,s,d", [(128, 2048, 64), (8, 1000, 128)])
def test_rope_bf16(cuda, bh, s, d):
    x = O.bf16_round(randn(2, bh, s, d))
    want = O.rope(x, f32_ln(5e5))
    got = host(ops.rope(dev(x, torch.bfloat16), 5e5))
    assert bf16_close(got, want)


@pytest.mark.parametrize("bh,s,d", [(32, 2048, 64), (8, 1000, 128), (2, 16384, 128)])
def test_rope_bf16_bwd(cuda, bh, s, d):
    """rope_backward (src/kernels/rope.rs:104-140) on bf16 gradients: within
    one bf16 rounding of the oracle on the same rounded input."""
    dy = O.bf16_round(randn(17, bh, s, d))
    want = O.rope(dy, f32_ln(5e5), backward=True)
    got = host(ops.rope(dev(dy, torch.bfloat16), 5e5, backward=True))
    assert bf16_close(got, want)


# ---------------------------------------------------------------------------
# Head transposes (bit-exact)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("b,s,h,d", [(4, 2048, 32, 64), (1, 37, 3, 8), (2, 129, 8, 128)])
def test_transpose_merge_bit_exact(cuda, dtype, b, s, h, d):
    x = randn(3, b, s, h * d)
    xd = dev(x, dtype)
    xb = xd.view(torch.int16 if dtype == torch.bfloat16 else torch.int32).cpu().numpy()
    t = ops.transpose_heads(xd, h)
    want = O.transpose_heads(xb, b, s, h, d)
    tb = t.view(torch.int16 if dtype == torch.bfloat16 else torch.int32).cpu().numpy()
    assert np.array_equal(tb, want)
    m = ops.merge_heads(t)
    assert torch.equal(m, xd)


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------

def test_fused_add_rmsnorm_reference_fixture(cuda):
    m, n = 4, 16
    x = O.load_fixture("fused_add_rmsnorm/input_x.bin").reshape(m, n)
    r = O.load_fixture("fused_add_rmsnorm/input_residual.bin").reshape(m, n)
    w = O.load_fixture("fused_add_rmsnorm/weight.bin")
    y, h, _ = ops.fused_add_rmsnorm(dev(x), dev(r), dev(w), 1e-6)
    assert np.abs(host(y) - O.load_fixture("fused_add_rmsnorm/output_y.bin").reshape(m, n)).max() < 1e-6
    assert np.array_equal(host(h), O.load_fixture("fused_add_rmsnorm/output_h.bin").reshape(m, n))


@pytest.mark.parametrize("m,n", [(8192, 2048), (37, 4096), (5, 24), (3, 1000)])
def test_rmsnorm_f32_fwd_bwd(cuda, m, n):
    x, r, w, g = randn(4, m, n), randn(5, m, n), randn(6, n), randn(7, m, n)
    y, h, rstd = ops.fused_add_rmsnorm(dev(x), dev(r), dev(w), 1e-5)
    ye, he, re_ = O.fused_add_rmsnorm_fwd(x, r, w, 1e-5)
    assert f32_close(host(y), ye)
    assert np.array_equal(host(h), he)
    assert np.abs(host(rstd) - re_).max() <= 1e-5 * np.abs(re_).max()
    # reference-formula fused backward
    dw0 = randn(8, n)
    dx, dres, dw = ops.fused_add_rmsnorm_bwd(dev(g), h, dev(w), rstd, dweight=dev(dw0))
    dxe, _, dwe = O.fused_add_rmsnorm_bwd(g, he, w, re_, dw_in=dw0)
    assert f32_close(host(dx), dxe)
    assert torch.equal(dx, dres)
    assert np.abs(host(dw) - dwe).max() <= 1e-5 * max(1.0, np.abs(dwe).max())
    # true-gradient plain backward
    yp, rp = ops.rmsnorm(dev(x), dev(w), 1e-5)
    dxp, dwp = ops.rmsnorm_bwd(dev(g), dev(x), dev(w), rp)
    dxpe, dwpe = O.rmsnorm_bwd(g, x, w, O.rmsnorm_fwd(x, w, 1e-5)[1])
    assert f32_close(host(dxp), dxpe)
    assert np.abs(host(dwp) - dwpe).max() <= 1e-5 * max(1.0, np.abs(dwpe).max())


@pytest.mark.parametrize("m,n", [(8192, 2048), (100, 4096), (16, 8192), (1, 1024)])
def test_rmsnorm_bf16(cuda, m, n):
    x = O.bf16_round(randn(9, m, n))
    r = O.bf16_round(randn(10, m, n))
    w = O.bf16_round(1 + 0.1 * randn(11, n))
    y, h, rstd = ops.fused_add_rmsnorm(dev(x, torch.bfloat16), dev(r, torch.bfloat16),
                                       dev(w, torch.bfloat16), 1e-5)
    ye, he, _ = O.fused_add_rmsnorm_fwd(x, r, w, 1e-5)
    assert np.array_equal(host(h), O.bf16_round(he))
    # y is computed from the bf16-rounded h (the reference reloads h), so
    # compare against the oracle on that h
    y2, _ = O.rmsnorm_fwd(O.bf16_round(he), w, 1e-5)
    err = np.abs(host(y) - y2)
    assert np.all(err <= np.abs(y2) * 2.0 ** -7 + 1e-2 * 2.0 ** -7)


def bf16_grad_close(got, want):
    """A bf16 gradient against the oracle's fp32 one on the same rounded
    inputs: one bf16 rounding, plus 1e-5 of the tensor's scale for the fp32
    row sums (dot(dy, w h), the weight gradient's sum over rows) that the
    kernel and the oracle add in different orders."""
    return np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -8 + 1e-5 * np.abs(want).max())


@pytest.mark.parametrize("m,n", [(8192, 2048), (100, 4096), (3, 1000)])
def test_rmsnorm_bf16_bwd(cuda, m, n):
    """bf16 backward of the fused add+RMSNorm (the reference's formula,
    src/kernels/fused_add_rmsnorm.rs:128-190) and of the plain norm (true
    gradient), rstd from the GPU forward as the backward receives it."""
    h = O.bf16_round(randn(18, m, n))
    w = O.bf16_round(1 + 0.1 * randn(19, n))
    g = O.bf16_round(randn(20, m, n))
    hd, wd, gd = dev(h, torch.bfloat16), dev(w, torch.bfloat16), dev(g, torch.bfloat16)
    _, rstd = ops.rmsnorm(hd, wd, 1e-5)
    r = host(rstd)
    assert np.abs(r - O.rmsnorm_fwd(h, w, 1e-5)[1]).max() <= 1e-5 * np.abs(r).max()
    dx, dres, dw = ops.fused_add_rmsnorm_bwd(gd, hd, wd, rstd)
    dxe, _, dwe = O.fused_add_rmsnorm_bwd(g, h, w, r)
    assert bf16_grad_close(host(dx), dxe)
    assert torch.equal(dx, dres)
    assert bf16_grad_close(host(dw), dwe)
    dxp, dwp = ops.rmsnorm_bwd(gd, hd, wd, rstd)
    dxpe, dwpe = O.rmsnorm_bwd(g, h, w, r)
    assert bf16_grad_close(host(dxp), dxpe)
    assert bf16_grad_close(host(dwp), dwpe)


# ---------------------------------------------------------------------------
# SwiGLU
# ---------------------------------------------------------------------------

def test_swiglu_reference_fixture(cuda):
    z = O.load_fixture("swiglu/input.bin").reshape(4, 16)
    got = host(ops.swiglu(dev(z)))
    assert np.abs(got - O.load_fixture("swiglu/output.bin").reshape(4, 8)).max() < 1e-6


@pytest.mark.parametrize("m,f", [(4096, 8192), (33, 100), (7, 12)])
def test_swiglu_f32(cuda, m, f):
    z, g = randn(12, m, 2 * f), randn(13, m, f)
    assert np.abs(host(ops.swiglu(dev(z))) - O.swiglu_fwd(z)).max() <= F32_TOL
    assert np.abs(host(ops.swiglu_bwd(dev(g), dev(z))) - O.swiglu_bwd(g, z)).max() <= F32_TOL


def test_swiglu_bf16(cuda):
    z = O.bf16_round(randn(14, 2048, 2 * 8192))
    got = host(ops.swiglu(dev(z, torch.bfloat16)))
    assert bf16_close(got, O.swiglu_fwd(z))


@pytest.mark.parametrize("m,f", [(2048, 8192), (33, 100)])
def test_swiglu_bf16_bwd(cuda, m, f):
    """swiglu_backward (src/kernels/swiglu.rs:97-136) on bf16: dz within one
    bf16 rounding of the oracle on the same rounded inputs."""
    z = O.bf16_round(randn(21, m, 2 * f))
    g = O.bf16_round(randn(22, m, f))
    got = host(ops.swiglu_bwd(dev(g, torch.bfloat16), dev(z, torch.bfloat16)))
    assert bf16_close(got, O.swiglu_bwd(g, z))


# ---------------------------------------------------------------------------
# Embedding gather (bit-exact)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_token_embed(cuda, dtype):
    V, Dm, S = 1000, 4096, 513
    w = dev(randn(15, V, Dm), dtype)
    ids = np.random.default_rng(16).integers(0, V, S)
    got_f = ops.token_embed(dev(ids.astype(np.float32)), w)  # the reference's f32 ids
    got_i = ops.token_embed(torch.from_numpy(ids.astype(np.int32)).cuda(), w)
    want = w[torch.from_numpy(ids).cuda()]
    assert torch.equal(got_f, want) and torch.equal(got_i, want)
    bad = ops.token_embed(torch.tensor([-1, V, 3], dtype=torch.int32, device="cuda"), w)
    assert torch.equal(bad[0], torch.zeros_like(bad[0])) and torch.equal(bad[2], w[3])


# ---------------------------------------------------------------------------
# Residual add (bit-exact: one fp32 add of the stored values, rounded once)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n", [8192 * 2048, 1001, 8])
def test_residual_add(cuda, dtype, n):
    a = dev(randn(23, n), dtype)
    b = dev(randn(24, n), dtype)
    want = (a.float() + b.float()).to(dtype)  # exact fp32 sum of two bf16/fp32 values, rounded
    assert torch.equal(ops.add(a, b), want)
    assert torch.equal(ops.add(a, b, out=a), want)  # in place

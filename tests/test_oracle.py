"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the parity reference.

Each oracle function is checked against the reference's own golden fixtures
(tests/golden/, copied from the reference's tests/fixtures) at the
reference's tolerance (tests/kernel_execution.rs:36), and, where no fixture
exists, against mathematics: fp64 dense attention, central finite
differences, closed forms, inverse pairs and brute force on tiny inputs.
"""
import json
import math
import os

import numpy as np
import pytest

from oracle import oracle as O

REF_TOL = 1e-4  # tests/kernel_execution.rs:36
GOLD = O.GOLDEN


def f32_ln(x):
    return float(np.log(np.float32(x)).astype(np.float32))


def rng(seed=0):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------------------
# RoPE
# ---------------------------------------------------------------------------

def test_rope_matches_reference_fixture():
    meta = json.load(open(os.path.join(GOLD, "rope", "meta.json")))
    bh, s, d = meta["bh"], meta["s"], meta["head_dim"]
    x = O.load_fixture("rope/input.bin").reshape(bh, s, d)
    y = O.load_fixture("rope/output.bin").reshape(bh, s, d)
    got = O.rope(x, f32_ln(meta["rope_base"]))
    err = np.abs(got - y).max()
    assert err < REF_TOL
    assert err < 1e-6  # observed 1.2e-7


@pytest.mark.parametrize("d,base", [(16, 1e4), (64, 1e4), (128, 5e5)])
def test_rope_closed_form(d, base):
    # y = R(theta) x with theta = pos * base^(-2k/d), interleaved pairs
    # (tests/fixtures/generate.py:43-66), float64, positions < 64.
    x = rng(1).standard_normal((3, 64, d)).astype(np.float32)
    got = O.rope(x, f32_ln(base))
    k = np.arange(d // 2, dtype=np.float64)
    theta = np.arange(64, dtype=np.float64)[:, None] * base ** (-2 * k / d)[None, :]
    c, s = np.cos(theta), np.sin(theta)
    xe, xo = x[..., 0::2].astype(np.float64), x[..., 1::2].astype(np.float64)
    want = np.stack([xe * c - xo * s, xe * s + xo * c], axis=-1).reshape(x.shape)
    assert np.abs(got - want).max() < 5e-5


def test_rope_inverse_and_invariants():
    x = rng(2).standard_normal((4, 300, 64)).astype(np.float32)
    lnb = f32_ln(5e5)
    y = O.rope(x, lnb)
    assert np.array_equal(y[:, 0], x[:, 0])  # position 0 is the identity
    back = O.rope(y, lnb, backward=True)
    assert np.abs(back - x).max() < 2e-6  # R(-t) R(t) = I
    n_x = x[..., 0::2] ** 2 + x[..., 1::2] ** 2
    n_y = y[..., 0::2] ** 2 + y[..., 1::2] ** 2
    assert np.abs(n_x - n_y).max() < 1e-4  # rotations keep each pair's norm


def test_rope_start_position():
    """orc_rope_at (rows of a slice at positions pos0, pos0 + 1, ...): bit for
    bit orc_rope of the same rows placed after pos0 zero rows, and the float64
    closed form at positions 515..518 (a KV-cached decode step's rows)."""
    x = rng(3).standard_normal((6, 4, 128)).astype(np.float32)
    lnb = f32_ln(5e5)
    for pos0 in (1, 37, 515):
        pad = np.concatenate([np.zeros((6, pos0, 128), np.float32), x], axis=1)
        for bwd in (False, True):
            want = O.rope(pad, lnb, backward=bwd)[:, pos0:]
            assert np.array_equal(O.rope(x, lnb, backward=bwd, pos0=pos0), want)
    got = O.rope(x, lnb, pos0=515)
    k = np.arange(64, dtype=np.float64)
    theta = np.arange(515, 519, dtype=np.float64)[:, None] * 5e5 ** (-2 * k / 128)[None, :]
    c, s_ = np.cos(theta), np.sin(theta)
    xe, xo = x[..., 0::2].astype(np.float64), x[..., 1::2].astype(np.float64)
    want = np.stack([xe * c - xo * s_, xe * s_ + xo * c], axis=-1).reshape(x.shape)
    assert np.abs(got - want).max() < 2e-4  # fp32 theta at position ~500: |dtheta| ~ 3e-5


def test_rope_inv_freq_rule():
    # inv = fp32(exp(fp32(k) * fp32(-2 ln b / d))), the rope.rs:88 operation order
    d, lnb = 128, f32_ln(5e5)
    c = np.float32(np.float32(-2.0) * np.float32(lnb)) / np.float32(d)
    want = np.array([np.float32(math.exp(float(np.float32(k) * c))) for k in range(d // 2)],
                    np.float32)
    assert np.array_equal(O.rope_inv_freq(d, lnb), want)


# ---------------------------------------------------------------------------
# SwiGLU
# ---------------------------------------------------------------------------

def _swiglu64(z):
    f = z.shape[1] // 2
    g, u = z[:, :f], z[:, f:]
    return g / (1 + np.exp(-g)) * u


def test_swiglu_matches_reference_fixture():
    meta = json.load(open(os.path.join(GOLD, "swiglu", "meta.json")))
    m, f = meta["m"], meta["d_ff"]
    z = O.load_fixture("swiglu/input.bin").reshape(m, 2 * f)
    want = O.load_fixture("swiglu/output.bin").reshape(m, f)
    got = O.swiglu_fwd(z)
    assert np.abs(got - want).max() < REF_TOL
    assert np.abs(got - want).max() < 1e-6
    # the float64 forward used for finite differences below is pinned too
    assert np.abs(_swiglu64(z.astype(np.float64)) - want).max() < 1e-6


def test_swiglu_bwd_finite_differences():
    z = rng(3).standard_normal((5, 24))
    g = rng(4).standard_normal((5, 12))
    dz = O.swiglu_bwd(g.astype(np.float32), z.astype(np.float32))
    num = np.zeros_like(z)
    h = 1e-6
    for idx in np.ndindex(z.shape):
        zp, zm = z.copy(), z.copy()
        zp[idx] += h
        zm[idx] -= h
        num[idx] = ((_swiglu64(zp) * g).sum() - (_swiglu64(zm) * g).sum()) / (2 * h)
    assert np.abs(dz - num).max() < 2e-5


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------

def _fused64(x, r, w, eps):
    h = x + r
    return h / np.sqrt((h * h).mean(-1, keepdims=True) + eps) * w


def test_fused_add_rmsnorm_matches_reference_fixture():
    meta = json.load(open(os.path.join(GOLD, "fused_add_rmsnorm", "meta.json")))
    m, n, eps = meta["m"], meta["n"], meta["eps"]
    x = O.load_fixture("fused_add_rmsnorm/input_x.bin").reshape(m, n)
    r = O.load_fixture("fused_add_rmsnorm/input_residual.bin").reshape(m, n)
    w = O.load_fixture("fused_add_rmsnorm/weight.bin")
    y_ref = O.load_fixture("fused_add_rmsnorm/output_y.bin").reshape(m, n)
    h_ref = O.load_fixture("fused_add_rmsnorm/output_h.bin").reshape(m, n)
    y, h, rstd = O.fused_add_rmsnorm_fwd(x, r, w, eps)
    assert np.abs(y - y_ref).max() < REF_TOL and np.abs(y - y_ref).max() < 1e-6
    assert np.array_equal(h, h_ref)
    assert np.abs(_fused64(x.astype(np.float64), r, w, eps) - y_ref).max() < 1e-6


def test_rmsnorm_plain_is_fused_with_zero_residual():
    x = rng(5).standard_normal((7, 40)).astype(np.float32)
    w = rng(6).standard_normal(40).astype(np.float32)
    y1, r1 = O.rmsnorm_fwd(x, w, 1e-5)
    y2, _, r2 = O.fused_add_rmsnorm_fwd(x, np.zeros_like(x), w, 1e-5)
    assert np.array_equal(y1, y2) and np.array_equal(r1, r2)
    assert np.abs(y1 - _fused64(x.astype(np.float64), 0, w, 1e-5)).max() < 2e-6


def _norm_fd(x, r, w, g, eps, step=1e-6):
    def loss(xx, ww):
        return (_fused64(xx, r, ww, eps) * g).sum()

    ndx = np.zeros_like(x)
    for idx in np.ndindex(x.shape):
        xp, xm = x.copy(), x.copy()
        xp[idx] += step
        xm[idx] -= step
        ndx[idx] = (loss(xp, w) - loss(xm, w)) / (2 * step)
    ndw = np.zeros_like(w)
    for i in range(w.shape[0]):
        wp, wm = w.copy(), w.copy()
        wp[i] += step
        wm[i] -= step
        ndw[i] = (loss(x, wp) - loss(x, wm)) / (2 * step)
    return ndx, ndw


def test_rmsnorm_bwd_finite_differences():
    m, n, eps = 4, 16, 1e-6
    x = rng(7).standard_normal((m, n))
    r = rng(8).standard_normal((m, n))
    w = rng(9).standard_normal(n)
    g = rng(10).standard_normal((m, n))
    _, h, rstd = O.fused_add_rmsnorm_fwd(x, r, w, eps)
    dw_in = rng(11).standard_normal(n).astype(np.float32)
    dx, dw = O.rmsnorm_bwd(g.astype(np.float32), h, w.astype(np.float32), rstd, dw_in=dw_in)
    ndx, ndw = _norm_fd(x, r, w, g, eps)
    assert np.abs(dx - ndx).max() < 5e-5
    assert np.abs((dw - dw_in) - ndw).max() < 5e-5  # dweight is accumulated into


def test_fused_add_rmsnorm_bwd_reference_formula():
    # fused_add_rmsnorm.rs:184 computes rstd*w*(dy - h*rstd^2*dot/N): the true
    # gradient when w == 1 (checked by finite differences), and for general w
    # it differs from the true gradient exactly by the factor w on the
    # rstd^3 * h * dot / N term.
    m, n, eps = 4, 16, 1e-6
    x = rng(7).standard_normal((m, n))
    r = rng(8).standard_normal((m, n))
    g = rng(10).standard_normal((m, n))
    ones = np.ones(n)
    _, h1, rstd1 = O.fused_add_rmsnorm_fwd(x, r, ones, eps)
    dx1, dres1, dw1 = O.fused_add_rmsnorm_bwd(g.astype(np.float32), h1, ones, rstd1)
    ndx, ndw = _norm_fd(x, r, ones, g, eps)
    assert np.abs(dx1 - ndx).max() < 5e-5
    assert np.array_equal(dx1, dres1)
    assert np.abs(dw1 - ndw).max() < 5e-5

    w = rng(9).standard_normal(n)
    _, h, rstd = O.fused_add_rmsnorm_fwd(x, r, w, eps)
    dxf, _, dwf = O.fused_add_rmsnorm_bwd(g.astype(np.float32), h, w.astype(np.float32), rstd)
    dxt, dwt = O.rmsnorm_bwd(g.astype(np.float32), h, w.astype(np.float32), rstd)
    h64, rs64 = h.astype(np.float64), rstd.astype(np.float64)[:, None]
    dot = (g * w * h64).sum(-1, keepdims=True)
    assert np.abs((dxf - dxt) - (-(w - 1) * rs64 ** 3 * h64 * dot / n)).max() < 2e-5
    assert np.array_equal(dwf, dwt)


# ---------------------------------------------------------------------------
# Flash attention
# ---------------------------------------------------------------------------

def _np_attention(q, k, v, scale, causal):
    """Brute-force float64 attention in numpy (independent of oracle.c)."""
    B, Hq, Sq, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    o = np.zeros((B, Hq, Sq, D))
    lse = np.zeros((B, Hq, Sq))
    for b in range(B):
        for h in range(Hq):
            kh = h // (Hq // Hkv)
            s = q[b, h].astype(np.float64) @ k[b, kh].astype(np.float64).T * scale
            if causal:
                s = np.where(np.arange(Sk)[None, :] > np.arange(Sq)[:, None], -np.inf, s)
            mx = s.max(-1, keepdims=True)
            e = np.exp(s - mx)
            o[b, h] = e / e.sum(-1, keepdims=True) @ v[b, kh].astype(np.float64)
            lse[b, h] = (mx + np.log(e.sum(-1, keepdims=True)))[:, 0]
    return o, lse


def _qkv(seed, B, Hq, Hkv, Sq, Sk, D):
    r = rng(seed)
    q = r.standard_normal((B, Hq, Sq, D)).astype(np.float32)
    k = r.standard_normal((B, Hkv, Sk, D)).astype(np.float32)
    v = r.standard_normal((B, Hkv, Sk, D)).astype(np.float32)
    return q, k, v


def test_dense_f64_matches_numpy_brute_force():
    for causal in (False, True):
        q, k, v = _qkv(12, 2, 4, 2, 9, 11, 8)
        r = O.attn_dense_f64(q, k, v, 0.3, causal)
        o, lse = _np_attention(q, k, v, 0.3, causal)
        assert np.abs(r["o"] - o).max() < 1e-12
        assert np.abs(r["lse"] - lse).max() < 1e-12


SHAPES = [  # B, Hq, Hkv, Sq, Sk, D
    (1, 4, 4, 128, 128, 64),   # the reference's case: fp32, no batch, MHA
    (2, 4, 2, 37, 37, 16),     # batch + GQA + ragged
    (1, 2, 1, 19, 33, 8),      # Sq != Sk (cross attention)
    (1, 2, 2, 70, 50, 32),     # Sq > Sk
]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("causal", [False, True])
def test_fa2_fwd_matches_dense_f64(shape, causal):
    B, Hq, Hkv, Sq, Sk, D = shape
    q, k, v = _qkv(13, *shape)
    scale = 1.0 / math.sqrt(D)
    o, lse = O.fa2_fwd(q, k, v, scale, causal)
    r = O.attn_dense_f64(q, k, v, scale, causal)
    assert np.abs(o - r["o"]).max() < 1e-5
    assert np.abs(lse - r["lse"]).max() < 1e-5
    o2, lse2 = O.fa2_fwd(q, k, v, scale, causal, all_keys=True)
    assert np.array_equal(o, o2) and np.array_equal(lse, lse2)


def test_fa2_fwd_invariants():
    q, k, v = _qkv(14, 1, 2, 2, 40, 40, 16)
    o, _ = O.fa2_fwd(q, k, v, 0.25, causal=True)
    assert np.abs(o[:, :, 0] - v[:, :, 0]).max() < 1e-6  # row 0 sees only key 0
    lo, hi = v.min(axis=2, keepdims=True), v.max(axis=2, keepdims=True)
    assert np.all(o >= lo - 1e-5) and np.all(o <= hi + 1e-5)  # convex combinations of V


@pytest.mark.parametrize("shape", SHAPES[1:])
@pytest.mark.parametrize("causal", [False, True])
def test_fa2_bwd_matches_dense_f64(shape, causal):
    B, Hq, Hkv, Sq, Sk, D = shape
    q, k, v = _qkv(15, *shape)
    do = rng(16).standard_normal(q.shape).astype(np.float32)
    scale = 1.0 / math.sqrt(D)
    o, lse = O.fa2_fwd(q, k, v, scale, causal)
    dq, dk, dv = O.fa2_bwd(q, k, v, o, do, lse, scale, causal)
    r = O.attn_dense_f64(q, k, v, scale, causal, do=do)
    for got, want in ((dq, r["dq"]), (dk, r["dk"]), (dv, r["dv"])):
        assert np.abs(got - want).max() < 2e-5


@pytest.mark.parametrize("causal", [False, True])
def test_dense_f64_grads_finite_differences(causal):
    q, k, v = _qkv(17, 1, 2, 1, 6, 6, 4)
    do = rng(18).standard_normal(q.shape).astype(np.float32)
    r = O.attn_dense_f64(q, k, v, 0.5, causal, do=do)
    step = 1e-3

    def loss(qq, kk, vv):
        o, _ = _np_attention(qq, kk, vv, 0.5, causal)
        return (o * do).sum()

    for name, t in (("dq", q), ("dk", k), ("dv", v)):
        t64 = t.astype(np.float64)
        num = np.zeros_like(t64)
        for idx in np.ndindex(t.shape):
            tp, tm = t64.copy(), t64.copy()
            tp[idx] += step
            tm[idx] -= step
            args_p = [tp if x is t else x.astype(np.float64) for x in (q, k, v)]
            args_m = [tm if x is t else x.astype(np.float64) for x in (q, k, v)]
            num[idx] = (loss(*args_p) - loss(*args_m)) / (2 * step)
        assert np.abs(r[name] - num).max() < 1e-5, name


# ---------------------------------------------------------------------------
# Blocks: the reference's encoder/decoder fixtures (RoPE disabled there)
# ---------------------------------------------------------------------------

def _load_block(name):
    meta = json.load(open(os.path.join(GOLD, name, "meta.json")))
    w = {k: O.load_fixture(f"{name}/{k.replace('.', '_')}.bin").reshape(s)
         for k, s in meta["weights"].items()}
    return meta, w


def _attn_oracle(xq, xkv, wq, wk, wv, wo, H, causal):
    Sq, Dm = xq.shape
    Sk = xkv.shape[0]
    Dh = Dm // H
    q = O.transpose_heads(xq @ wq.T, 1, Sq, H, Dh)
    k = O.transpose_heads(xkv @ wk.T, 1, Sk, H, Dh)
    v = O.transpose_heads(xkv @ wv.T, 1, Sk, H, Dh)
    o, _ = O.fa2_fwd(q, k, v, 1.0 / math.sqrt(Dh), causal)
    return O.transpose_heads(o, 1, Sq, H, Dh, merge=True)[0] @ wo.T


def test_encoder_block_fixture_composition():
    meta, w = _load_block("encoder_block")
    x = O.load_fixture("encoder_block/input.bin").reshape(meta["seq"], meta["d_model"])
    H, eps = meta["n_heads"], 1e-6  # generate.py:136
    n1, _ = O.rmsnorm_fwd(x, w["norm1.weight"], eps)
    x2 = x + _attn_oracle(n1, n1, w["wq.weight"], w["wk.weight"], w["wv.weight"],
                          w["wo.weight"], H, causal=False)
    n2, _ = O.rmsnorm_fwd(x2, w["norm2.weight"], eps)
    out = x2 + O.swiglu_fwd(n2 @ w["wgate_up.weight"].T) @ w["wdown.weight"].T
    want = O.load_fixture("encoder_block/output.bin").reshape(out.shape)
    assert np.abs(out - want).max() < 1e-5


def test_decoder_block_fixture_composition():
    meta, w = _load_block("decoder_block")
    st, se, Dm = meta["seq_tgt"], meta["seq_enc"], meta["d_model"]
    tgt = O.load_fixture("decoder_block/input_tgt.bin").reshape(st, Dm)
    enc = O.load_fixture("decoder_block/input_enc.bin").reshape(se, Dm)
    H, eps = meta["n_heads"], 1e-6
    n1, _ = O.rmsnorm_fwd(tgt, w["norm1.weight"], eps)
    t = tgt + _attn_oracle(n1, n1, w["wqs.weight"], w["wks.weight"], w["wvs.weight"],
                           w["wos.weight"], H, causal=True)
    n2, _ = O.rmsnorm_fwd(t, w["norm2.weight"], eps)
    t = t + _attn_oracle(n2, enc, w["wqc.weight"], w["wkc.weight"], w["wvc.weight"],
                         w["woc.weight"], H, causal=False)
    n3, _ = O.rmsnorm_fwd(t, w["norm3.weight"], eps)
    out = t + O.swiglu_fwd(n3 @ w["wgate_up.weight"].T) @ w["wdown.weight"].T
    want = O.load_fixture("decoder_block/output.bin").reshape(out.shape)
    assert np.abs(out - want).max() < 1e-5


# ---------------------------------------------------------------------------
# Transpose and embedding: brute force
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [np.float32, np.uint16])
def test_transpose_heads_brute_force(dtype):
    B, S, H, Dh = 2, 5, 3, 4
    x = (rng(19).standard_normal((B, S, H * Dh)) * 1000).astype(dtype)
    t = O.transpose_heads(x, B, S, H, Dh)
    for b in range(B):
        for h in range(H):
            for s in range(S):
                # transpose_heads.rs:65-67: dst[h, s, d] = src[s, h*Dh + d]
                assert np.array_equal(t[b, h, s], x[b, s, h * Dh:(h + 1) * Dh])
    back = O.transpose_heads(t, B, S, H, Dh, merge=True)
    assert np.array_equal(back, x)


def test_token_embed_brute_force():
    w = rng(20).standard_normal((50, 12)).astype(np.float32)
    ids = np.array([3, 0, 49, 3, 17], np.float32)
    out = O.token_embed(ids, w)
    assert np.array_equal(out, w[ids.astype(int)])


# ---------------------------------------------------------------------------
# The reference-precision config: RoPE -> transpose -> causal FA2, fp32
# ---------------------------------------------------------------------------

def test_c1_pipeline_against_dense_f64():
    B, S, H, D = 1, 128, 4, 64
    r = rng(21)
    q_bshd = r.standard_normal((B, S, H * D)).astype(np.float32)
    k_bshd = r.standard_normal((B, S, H * D)).astype(np.float32)
    v_bshd = r.standard_normal((B, S, H * D)).astype(np.float32)
    lnb = f32_ln(1e4)
    q = O.rope(O.transpose_heads(q_bshd, B, S, H, D), lnb)
    k = O.rope(O.transpose_heads(k_bshd, B, S, H, D), lnb)
    v = O.transpose_heads(v_bshd, B, S, H, D)
    o, lse = O.fa2_fwd(q, k, v, 1.0 / 8.0, causal=True)
    ref = O.attn_dense_f64(q, k, v, 1.0 / 8.0, causal=True)
    assert np.abs(o - ref["o"]).max() < 1e-5
    assert np.abs(lse - ref["lse"]).max() < 1e-5


def test_fa2_q_offset_slices_are_exact():
    # a slice of query rows with q_offset reproduces those rows of the full
    # problem; keys at or past the slice start only see rows in the slice
    q, k, v = _qkv(22, 1, 2, 2, 64, 64, 16)
    do = rng(23).standard_normal(q.shape).astype(np.float32)
    o, l = O.fa2_fwd(q, k, v, 0.25, True)
    o2, l2 = O.fa2_fwd(q[:, :, 40:], k, v, 0.25, True, q_offset=40)
    assert np.array_equal(o[:, :, 40:], o2) and np.array_equal(l[:, :, 40:], l2)
    dq, dk, dv = O.fa2_bwd(q, k, v, o, do, l, 0.25, True)
    dq2, dk2, dv2 = O.fa2_bwd(q[:, :, 40:], k, v, o2, do[:, :, 40:], l2, 0.25, True, q_offset=40)
    assert np.array_equal(dq[:, :, 40:], dq2)
    assert np.array_equal(dk[:, :, 40:], dk2[:, :, 40:])
    assert np.array_equal(dv[:, :, 40:], dv2[:, :, 40:])

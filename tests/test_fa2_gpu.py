"""GPU parity of flash-attention 2 (forward and backward) against the oracle.

fp32 path: max abs <= 1e-5 against the oracle's fp32 restatement of the
reference kernels, for O, LSE and the gradients alike.  bf16 path: rel-L2 <= 5e-3 and max abs <= 2e-2 against
the fp32 oracle run on the same bf16-rounded inputs, for O and for the fp32
gradients of the bf16 backward (TEENY_GRAD_F32); gradients stored as bf16
get the same bar with the max-abs part scaled by the tensor's magnitude
above 4 (check_bf16); LSE (fp32) within 2e-2.  Each op is compared on its
own inputs: the backward's oracle receives the same O and LSE the GPU
backward received.  At the full benchmark shapes the GPU runs the whole
problem and the oracle checks every row and key of whole (batch, kv head)
groups.
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from teenyformers_amd import ops

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5
BF16_MAX_ABS = 2e-2
BF16_REL_L2 = 5e-3


def randn(seed, *shape):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def dev(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def host(t):
    return t.float().cpu().numpy()


def rel_l2(got, want):
    """||got - want|| / ||want||, or None when the reference is exactly zero:
    there the relative error is undefined and the max-abs bar alone applies
    (one query row and one key: O = V, so dP = Delta and dS, dQ and dK are
    exactly zero, and the kernels return rounding noise of ~1e-8)."""
    n = np.linalg.norm(want.ravel())
    return None if n == 0 else float(np.linalg.norm((got - want).ravel()) / n)


def bf16_bar(m):
    """The max-abs bar of a bf16-stored tensor whose largest value is m:
    2e-2 * max(1, 2^(floor(log2 m) - 1)).  2e-2 is 2.56 half-ulps of the
    bf16 binade [2, 4) (half-ulp 2^-7).  A bf16 value in the binade
    [2^e, 2^(e+1)) cannot sit closer than its half-ulp 2^(e-8) to the fp32
    value it stores, so a tensor whose largest values exceed 4 (GQA-summed
    dK/dV, dQ of the 8x-spiked keys: up to ~36) gets the same 2.56 half-ulps
    of its top binade; unit-scale tensors, such as every output at the B8 H32
    S4096 D128 shape, get the flat 2e-2."""
    return BF16_MAX_ABS * max(1.0, 2.0 ** (math.floor(math.log2(m)) - 1)) if m > 0 else BF16_MAX_ABS


def check_bf16(name, got, want):
    """bf16 bar: rel-L2 <= 5e-3 and max abs <= bf16_bar(max|want|)."""
    err = float(np.abs(got - want).max())
    r = rel_l2(got, want)
    bar = bf16_bar(float(np.abs(want).max()))
    assert err <= bar and (r is None or r <= BF16_REL_L2), \
        f"{name}: max abs {err:.3e} (bar {bar:.3e}), rel-L2 {r}"


def check_flat(name, got, want):
    """The stated bf16 bar without scaling: rel-L2 <= 5e-3, max abs <= 2e-2
    (for outputs that are not rounded to bf16: O's error is the bf16
    rounding of its own storage, but the fp32 gradients carry only the
    kernels' bf16 operand rounding)."""
    err = float(np.abs(got - want).max())
    r = rel_l2(got, want)
    assert err <= BF16_MAX_ABS and (r is None or r <= BF16_REL_L2), \
        f"{name}: max abs {err:.3e}, rel-L2 {r}"


def inputs(seed, B, Hq, Hkv, Sq, Sk, D, bf16, spike=False):
    q, k, v, do = (randn(seed, B, Hq, Sq, D), randn(seed + 1, B, Hkv, Sk, D),
                   randn(seed + 2, B, Hkv, Sk, D), randn(seed + 3, B, Hq, Sq, D))
    if spike:  # 1% of K rows x8 stresses the running max
        rows = np.random.default_rng(seed + 4).choice(Sk, max(1, Sk // 100), replace=False)
        k[:, :, rows] *= 8
    if bf16:
        q, k, v, do = (O.bf16_round(t) for t in (q, k, v, do))
    return q, k, v, do


# ---------------------------------------------------------------------------
# fp32: the reference's precision
# ---------------------------------------------------------------------------

def test_c1_rope_transpose_fa2_f32(cuda):
    """B1 H4 S128 D64: RoPE (theta 1e4) + [B,S,H,D]->[B,H,S,D] + causal FA2."""
    B, S, H, D = 1, 128, 4, 64
    qs, ks, vs = randn(100, B, S, H * D), randn(101, B, S, H * D), randn(102, B, S, H * D)
    lnb = float(np.log(np.float32(1e4)).astype(np.float32))
    q = ops.rope(ops.transpose_heads(dev(qs, torch.float32), H), 1e4)
    k = ops.rope(ops.transpose_heads(dev(ks, torch.float32), H), 1e4)
    v = ops.transpose_heads(dev(vs, torch.float32), H)
    o, lse = ops.flash_attn2_fwd(q, k, v, 1.0 / math.sqrt(D), causal=True)
    qe = O.rope(O.transpose_heads(qs, B, S, H, D), lnb)
    ke = O.rope(O.transpose_heads(ks, B, S, H, D), lnb)
    ve = O.transpose_heads(vs, B, S, H, D)
    oe, le = O.fa2_fwd(qe, ke, ve, 1.0 / math.sqrt(D), True)
    assert np.abs(host(o) - oe).max() <= F32_TOL
    assert np.abs(host(lse) - le).max() <= F32_TOL


F32_SHAPES = [  # B, Hq, Hkv, Sq, Sk, D
    (1, 4, 4, 128, 128, 64),
    (2, 4, 2, 77, 77, 32),
    (1, 2, 1, 40, 90, 16),
    (1, 2, 2, 90, 40, 128),
    (1, 3, 3, 65, 65, 8),
]


@pytest.mark.parametrize("shape", F32_SHAPES)
@pytest.mark.parametrize("causal", [True, False])
def test_fa2_f32_fwd_bwd(cuda, shape, causal):
    B, Hq, Hkv, Sq, Sk, D = shape
    q, k, v, do = inputs(10, *shape, bf16=False)
    scale = 1.0 / math.sqrt(D)
    qd, kd, vd, dod = (dev(t, torch.float32) for t in (q, k, v, do))
    o, lse = ops.flash_attn2_fwd(qd, kd, vd, scale, causal)
    oe, le = O.fa2_fwd(q, k, v, scale, causal)
    assert np.abs(host(o) - oe).max() <= F32_TOL
    assert np.abs(host(lse) - le).max() <= F32_TOL
    dq, dk, dv = ops.flash_attn2_bwd(qd, kd, vd, o, lse, dod, scale, causal)
    dqe, dke, dve = O.fa2_bwd(q, k, v, oe, do, le, scale, causal)
    for name, got, want in (("dq", dq, dqe), ("dk", dk, dke), ("dv", dv, dve)):
        err = float(np.abs(host(got) - want).max())
        print(f"fa2 f32 {shape} causal={causal} {name}: max abs {err:.2e} "
              f"(max |want| {np.abs(want).max():.2f})", flush=True)
        assert err <= F32_TOL, f"{name} {err}"


# ---------------------------------------------------------------------------
# bf16 MFMA path
# ---------------------------------------------------------------------------

BF16_SHAPES = [  # B, Hq, Hkv, Sq, Sk, D
    (1, 4, 4, 128, 128, 64),
    (2, 8, 2, 300, 300, 128),   # GQA 4, ragged
    (1, 8, 1, 513, 513, 128),   # GQA 8 (MQA), ragged past a tile
    (2, 4, 4, 256, 256, 64),
    (1, 4, 2, 100, 300, 128),   # Sq < Sk
    (1, 4, 2, 300, 100, 64),    # Sq > Sk
    (1, 2, 2, 1, 1, 64),        # one row
    (1, 2, 2, 1024, 1024, 128),
    (2, 8, 2, 200, 260, 64),    # causal: GQA 4 packed (a wavefront per q head), Sq < Sk
    (1, 8, 2, 300, 100, 64),    # GQA 4 packed, Sq > Sk
    (1, 16, 2, 333, 333, 128),  # GQA 8 packed
    (1, 4, 1, 1, 100, 64),      # GQA 4 packed, one query row
    (2, 8, 2, 33, 70, 128),     # GQA 4 packed, one row past a 32-row block
]


@pytest.mark.parametrize("shape", BF16_SHAPES)
@pytest.mark.parametrize("causal", [True, False])
def test_fa2_bf16_fwd(cuda, shape, causal):
    B, Hq, Hkv, Sq, Sk, D = shape
    q, k, v, _ = inputs(20, *shape, bf16=True, spike=True)
    scale = 1.0 / math.sqrt(D)
    o, lse = ops.flash_attn2_fwd(dev(q, torch.bfloat16), dev(k, torch.bfloat16),
                                 dev(v, torch.bfloat16), scale, causal)
    oe, le = O.fa2_fwd(q, k, v, scale, causal)
    check_bf16("O", host(o), oe)
    assert np.abs(host(lse) - le).max() <= 2e-2


MERGED_SHAPES = BF16_SHAPES + [
    (16, 32, 8, 512, 512, 128),    # the Llama-3-8B prefill's attention
    (1, 8, 8, 2048, 2048, 128),    # plain, several row blocks
    (1, 8, 2, 5000, 5000, 128),    # GQA 4 packed, long
]


@pytest.mark.parametrize("shape", MERGED_SHAPES)
@pytest.mark.parametrize("causal", [True, False])
def test_fa2_bf16_fwd_merged(cuda, shape, causal):
    """The merged-heads forward writes [B, Sq, Hq*D]: bit for bit
    merge_heads of the [B, Hq, Sq, D] forward, LSE bit for bit the same."""
    B, Hq, Hkv, Sq, Sk, D = shape
    g = torch.Generator(device="cuda").manual_seed(Sq * 7 + Hq)
    q = torch.randn((B, Hq, Sq, D), generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn((B, Hkv, Sk, D), generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn((B, Hkv, Sk, D), generator=g, device="cuda").to(torch.bfloat16)
    scale = 1.0 / math.sqrt(D)
    o, lse = ops.flash_attn2_fwd(q, k, v, scale, causal)
    om, lm = ops.flash_attn2_fwd_merged(q, k, v, scale, causal)
    torch.cuda.synchronize()
    assert om.shape == (B, Sq, Hq * D)
    assert torch.equal(om.view(torch.int16), ops.merge_heads(o).view(torch.int16))
    assert torch.equal(lm.view(torch.int32), lse.view(torch.int32))


QKV_SHAPES = [  # B, Hq, Hkv, S, cache length, D
    (16, 32, 8, 512, 640, 128),   # the Llama-3-8B prefill (GQA 4 packed)
    (4, 32, 8, 2048, 2048, 64),   # the Llama block
    (2, 8, 8, 300, 320, 128),     # MHA: the 4-wavefront form, ragged
    (1, 16, 2, 333, 400, 128),    # GQA 8 packed
    (1, 8, 2, 8200, 8200, 128),   # the 8-wavefront form (8000+ rows)
    (3, 4, 1, 1, 64, 64),         # one prompt row
]


@pytest.mark.parametrize("shape", QKV_SHAPES)
@pytest.mark.parametrize("causal", [True, False])
def test_fa2_bf16_fwd_qkv(cuda, shape, causal):
    """The prompt attention from the fused QKV projection (its q heads
    rotated as they load, with the RoPE table's (cos, sin)) gives the bits of
    the split into a Q buffer followed by the merged-heads forward; the split
    without q_out writes the same cache rows and nothing else."""
    B, Hq, Hkv, S, L, D = shape
    base = 5e5
    g = torch.Generator(device="cuda").manual_seed(S + Hq + D)
    qkv = torch.randn((B, S, (Hq + 2 * Hkv) * D), generator=g, device="cuda").to(torch.bfloat16)
    kc1 = torch.zeros((B, Hkv, L, D), dtype=torch.bfloat16, device="cuda")
    vc1, kc2, vc2 = torch.zeros_like(kc1), torch.zeros_like(kc1), torch.zeros_like(kc1)
    q = torch.empty((B, Hq, S, D), dtype=torch.bfloat16, device="cuda")
    ops.qkv_rope_split(qkv, q, kc1, vc1, 0, Hq, Hkv, base)
    ops.qkv_rope_split(qkv, None, kc2, vc2, 0, Hq, Hkv, base)
    scale = 1.0 / math.sqrt(D)
    o1, l1 = ops.flash_attn2_fwd_merged(q, kc1, vc1, scale, causal)
    cs = ops.rope_table(S + 3, D, base, "cuda")
    o2, l2 = ops.flash_attn2_fwd_qkv(qkv, cs, kc2, vc2, Hq, scale, causal)
    torch.cuda.synchronize()
    assert torch.equal(kc1.view(torch.int16), kc2.view(torch.int16))
    assert torch.equal(vc1.view(torch.int16), vc2.view(torch.int16))
    assert torch.equal(o2.view(torch.int16), o1.view(torch.int16))
    assert torch.equal(l2.view(torch.int32), l1.view(torch.int32))


def test_rope_table_values(cuda):
    """teeny_rope_table against the angle of rope.rs:86-88 formed as the
    oracle forms it (fp32 theta = fp32(pos) * fp32(exp(fp32(k * c)))), its
    cos and sin taken in float64: within a few fp32 ulps of 1."""
    n, D, base = 4100, 128, 5e5
    cs = ops.rope_table_pairs(ops.rope_table(n, D, base, "cuda"), D).cpu().numpy()
    assert cs.shape == (4128, D // 2, 2)
    cs = cs[:n].astype(np.float64)
    c = np.float32(np.float32(-2.0) * np.float32(ops._ln(base))) / np.float32(D)
    kc = (np.arange(D // 2, dtype=np.float32) * c).astype(np.float64)
    inv = np.exp(kc).astype(np.float32)
    theta = (np.arange(n, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float64)
    err = np.maximum(np.abs(cs[..., 0] - np.cos(theta)), np.abs(cs[..., 1] - np.sin(theta)))
    assert float(err.max()) <= 2.5e-7, float(err.max())


def test_fa2_fwd_merged_rejects_f32(cuda):
    q = torch.zeros((1, 2, 8, 64), device="cuda")
    with pytest.raises(TypeError):
        ops.flash_attn2_fwd_merged(q, q, q)


@pytest.mark.parametrize("B,Hq,Hkv,S,D", [(1, 8, 2, 8300, 64), (1, 8, 2, 5000, 128)])
def test_fa2_bf16_fwd_packed_long(cuda, B, Hq, Hkv, S, D):
    """The GQA-packed causal forward (a wavefront per q head of a group of
    4) on long sequences: D = 64 takes it at any length, D = 128 below 8000
    rows.  The first, a middle and the last 128 query rows of every head
    against the oracle (q_offset gives the slice its causal positions)."""
    q, k, v, _ = inputs(80 + S, B, Hq, Hkv, S, S, D, bf16=True, spike=True)
    scale = 1.0 / math.sqrt(D)
    o, lse = ops.flash_attn2_fwd(dev(q, torch.bfloat16), dev(k, torch.bfloat16),
                                 dev(v, torch.bfloat16), scale, True)
    o, lse = host(o), host(lse)
    for r0 in (0, S // 2 + 5, S - 128):
        oe, le = O.fa2_fwd(q[:, :, r0:r0 + 128], k, v, scale, True, q_offset=r0)
        check_bf16(f"O rows {r0}+", o[:, :, r0:r0 + 128], oe)
        assert np.abs(lse[:, :, r0:r0 + 128] - le).max() <= 2e-2


@pytest.mark.parametrize("causal", [True, False])
def test_fa2_bf16_fwd_late_maximum(cuda, causal):
    """Rows whose maximum score lies far past their first 64-key tile: keys
    150-159 scaled x30 and key 300 x60 put P = 2^(t - m) of the first tile's
    maximum m beyond 2^31 (and beyond fp32 for key 300), so the forward must
    redo those tiles with their own maximum and rescale O and l; O and LSE
    as the oracle's."""
    B, Hq, Hkv, S, D = 1, 4, 2, 384, 128
    q, k, v, _ = inputs(31, B, Hq, Hkv, S, S, D, bf16=True)
    k[:, :, 150:160] *= 30
    k[:, :, 300] *= 60
    k = O.bf16_round(k)
    scale = 1.0 / math.sqrt(D)
    o, lse = ops.flash_attn2_fwd(dev(q, torch.bfloat16), dev(k, torch.bfloat16),
                                 dev(v, torch.bfloat16), scale, causal)
    oe, le = O.fa2_fwd(q, k, v, scale, causal)
    assert np.isfinite(host(o)).all() and np.isfinite(host(lse)).all()
    check_bf16("O", host(o), oe)
    assert np.abs(host(lse) - le).max() <= 2e-2 * max(1.0, float(np.abs(le).max()) / 64)


@pytest.mark.parametrize("shape", BF16_SHAPES)
@pytest.mark.parametrize("causal", [True, False])
def test_fa2_bf16_bwd(cuda, shape, causal):
    B, Hq, Hkv, Sq, Sk, D = shape
    q, k, v, do = inputs(30, *shape, bf16=True)
    scale = 1.0 / math.sqrt(D)
    qd, kd, vd, dod = (dev(t, torch.bfloat16) for t in (q, k, v, do))
    o, lse = ops.flash_attn2_fwd(qd, kd, vd, scale, causal)
    dq, dk, dv = ops.flash_attn2_bwd(qd, kd, vd, o, lse, dod, scale, causal)
    # the backward op's inputs include O and LSE: the oracle gets the same ones
    dqe, dke, dve = O.fa2_bwd(q, k, v, host(o), do, host(lse), scale, causal)
    check_bf16("dQ", host(dq), dqe)
    check_bf16("dK", host(dk), dke)
    check_bf16("dV", host(dv), dve)
    # fp32 gradients from the same kernels: the flat bar
    g32 = ops.flash_attn2_bwd(qd, kd, vd, o, lse, dod, scale, causal, grad_f32=True)
    assert all(t.dtype == torch.float32 for t in g32)
    for name, got, want in zip(("dQ", "dK", "dV"), g32, (dqe, dke, dve)):
        check_flat(name + " (fp32)", host(got), want)
    # the hi + lo operands leave the fp32 gradients closer to the oracle
    for a, b, w in zip(g32, (dq, dk, dv), (dqe, dke, dve)):
        ra, rb = rel_l2(host(a), w), rel_l2(host(b), w)
        assert ra is None or ra <= rb


@pytest.mark.parametrize("shape", [(1, 4, 2, 2048, 2048, 64), (1, 2, 1, 2100, 2050, 128),
                                   (2, 4, 2, 2200, 2200, 64)])
def test_fa2_bf16_bwd_gqa_two_groups(cuda, shape):
    """Causal GQA with an even group and 2048+ query rows: dK/dV in two
    wavefront groups per workgroup, each walking half of the q heads of the
    same keys, their sums added through LDS; no partial sums, so the larger
    workspace equals the base one.  bf16 and fp32 gradients against the
    oracle."""
    B, Hq, Hkv, Sq, Sk, D = shape
    q, k, v, do = inputs(50, *shape, bf16=True)
    scale = 1.0 / math.sqrt(D)
    qd, kd, vd, dod = (dev(t, torch.bfloat16) for t in (q, k, v, do))
    o, lse = ops.flash_attn2_fwd(qd, kd, vd, scale, True)
    assert ops.flash_attn2_bwd_workspace_bytes(qd, kd) == ops.flash_attn2_bwd_workspace_bytes(qd)
    dq, dk, dv = ops.flash_attn2_bwd(qd, kd, vd, o, lse, dod, scale, True)
    g32 = ops.flash_attn2_bwd(qd, kd, vd, o, lse, dod, scale, True, grad_f32=True)
    dqe, dke, dve = O.fa2_bwd(q, k, v, host(o), do, host(lse), scale, True)
    for name, got, w in zip(("dQ", "dK", "dV"), (dq, dk, dv), (dqe, dke, dve)):
        check_bf16(name, host(got), w)
    for name, got, w in zip(("dQ", "dK", "dV"), g32, (dqe, dke, dve)):
        check_flat(name + " (fp32)", host(got), w)


@pytest.mark.parametrize("grad_f32", [False, True])
def test_fa2_bf16_bwd_gqa_split(cuda, grad_f32):
    """B1 Hq2 Hkv1 S12288 D64 causal (a group of 2, 96 key blocks): with the
    workspace of teeny_flash_attn2_bwd_workspace_bytes_gqa each group's q
    heads split over 2 dK/dV workgroups (fp32 partials merged in a fixed
    order); with the base workspace the two-group kernel runs instead.  dQ
    is the same kernel either way; dK and dV agree to the bf16 rounding of
    the summation order (or closer, for fp32 gradients).  The split against
    the oracle: the B1 Hq64 Hkv8 S16384 whole-group test (4 splits)."""
    B, Hq, Hkv, S, D = 1, 2, 1, 12288, 64
    gen = torch.Generator(device="cuda").manual_seed(51)
    q, do = (torch.randn(B, Hq, S, D, generator=gen, device="cuda").to(torch.bfloat16)
             for _ in range(2))
    k, v = (torch.randn(B, Hkv, S, D, generator=gen, device="cuda").to(torch.bfloat16)
            for _ in range(2))
    scale = 1.0 / math.sqrt(D)
    o, lse = ops.flash_attn2_fwd(q, k, v, scale, True)
    small = ops.flash_attn2_bwd_workspace_bytes(q)
    big = ops.flash_attn2_bwd_workspace_bytes(q, k)
    assert big == small + 2 * 2 * B * Hkv * S * D * 4
    outs = []
    for n in (small, big):
        print(f"  workspace {n} bytes, grad_f32={grad_f32}", flush=True)
        ws = torch.empty(n, dtype=torch.uint8, device="cuda")
        outs.append(ops.flash_attn2_bwd(q, k, v, o, lse, do, scale, True, workspace=ws,
                                        grad_f32=grad_f32))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0])
    tol = 2.0 ** -20 if grad_f32 else 2.0 ** -7
    for a, b in ((outs[0][1], outs[1][1]), (outs[0][2], outs[1][2])):
        a, b = host(a), host(b)
        assert np.isfinite(a).all() and np.isfinite(b).all()
        assert np.all(np.abs(a - b) <= np.abs(a) * tol + 1e-6)


def _random_shapes(n, seed=2026):
    """Seeded random shapes off the tile grid: ragged lengths, Sq != Sk, GQA
    groups 1-8, both head dims."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        hkv = int(rng.choice([1, 2, 4]))
        group = int(rng.choice([1, 2, 4, 8]))
        sq = int(rng.integers(1, 700))
        sk = sq if rng.random() < 0.5 else int(rng.integers(1, 700))
        out.append((int(rng.integers(1, 4)), hkv * group, hkv, sq, sk, int(rng.choice([64, 128])),
                    bool(rng.random() < 0.6)))
    return out


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,D,causal", _random_shapes(12))
def test_fa2_bf16_random_shapes(cuda, B, Hq, Hkv, Sq, Sk, D, causal):
    """Forward and backward at seeded random shapes against the oracle."""
    q, k, v, do = inputs(60 + Sq, B, Hq, Hkv, Sq, Sk, D, bf16=True, spike=Sk >= 100)
    scale = 1.0 / math.sqrt(D)
    qd, kd, vd, dod = (dev(t, torch.bfloat16) for t in (q, k, v, do))
    o, lse = ops.flash_attn2_fwd(qd, kd, vd, scale, causal)
    oe, le = O.fa2_fwd(q, k, v, scale, causal)
    check_bf16("O", host(o), oe)
    finite = np.isfinite(le)  # causal rows with no visible key (Sq > Sk) have no LSE
    assert np.abs(host(lse)[finite] - le[finite]).max(initial=0.0) <= 2e-2
    dq, dk, dv = ops.flash_attn2_bwd(qd, kd, vd, o, lse, dod, scale, causal)
    dqe, dke, dve = O.fa2_bwd(q, k, v, host(o), do, host(lse), scale, causal)
    check_bf16("dQ", host(dq), dqe)
    check_bf16("dK", host(dk), dke)
    check_bf16("dV", host(dv), dve)
    # fp32 gradients from the same kernels (hi + lo bf16 P and dS): the flat bar
    g32 = ops.flash_attn2_bwd(qd, kd, vd, o, lse, dod, scale, causal, grad_f32=True)
    for name, got, want in zip(("dQ", "dK", "dV"), g32, (dqe, dke, dve)):
        check_flat(name + " (fp32)", host(got), want)


@pytest.mark.parametrize("B,Hq,Hkv,S,D", [(1, 8, 2, 700, 128), (3, 8, 2, 777, 128),
                                         (16, 32, 8, 512, 128), (2, 8, 8, 1000, 64)])
def test_fa2_bf16_deterministic(cuda, B, Hq, Hkv, S, D):
    """Every output bit-identical across calls: O, LSE, dQ, dK, dV (and
    the fp32-gradient option).  A row maximum that read a matrix product's
    result too early once made whole rows of O and LSE differ by an ulp
    from call to call at D = 128."""
    q, k, v, do = inputs(40 + S, B, Hq, Hkv, S, S, D, bf16=True)
    qd, kd, vd, dod = (dev(t, torch.bfloat16) for t in (q, k, v, do))
    runs = []
    for _ in range(3):
        o, lse = ops.flash_attn2_fwd(qd, kd, vd)
        g = ops.flash_attn2_bwd(qd, kd, vd, o, lse, dod)
        g32 = ops.flash_attn2_bwd(qd, kd, vd, o, lse, dod, grad_f32=True)
        runs.append((o, lse) + tuple(g) + tuple(g32))
    for other in runs[1:]:
        for name, x, y in zip(("O", "LSE", "dQ", "dK", "dV", "dQ32", "dK32", "dV32"),
                              runs[0], other):
            assert torch.equal(x, y), name


# ---------------------------------------------------------------------------
# Full benchmark shapes: whole (batch, kv head) groups against the oracle
# ---------------------------------------------------------------------------

def _group_check(B, Hq, Hkv, S, D, seed, spike, groups):
    """Run fwd+bwd at full size on the GPU, with bf16 and with fp32
    gradients; the oracle then evaluates every query row of each listed
    (b, kv head) group's q heads and every key of its kv head: O, LSE, dQ
    and the GQA-summed dK/dV, key block 0 (which accumulates every query
    row of every q head of the group) included."""
    gen = torch.Generator(device="cuda").manual_seed(seed)
    shape_q, shape_kv = (B, Hq, S, D), (B, Hkv, S, D)
    q = torch.randn(shape_q, generator=gen, device="cuda").to(torch.bfloat16)
    k = torch.randn(shape_kv, generator=gen, device="cuda")
    if spike:
        idx = torch.randperm(S, generator=gen, device="cuda")[: max(1, S // 100)]
        k[:, :, idx] *= 8
    k = k.to(torch.bfloat16)
    v = torch.randn(shape_kv, generator=gen, device="cuda").to(torch.bfloat16)
    do = torch.randn(shape_q, generator=gen, device="cuda").to(torch.bfloat16)
    scale = 1.0 / math.sqrt(D)
    o, lse = ops.flash_attn2_fwd(q, k, v, scale, True)
    dq, dk, dv = ops.flash_attn2_bwd(q, k, v, o, lse, do, scale, True)
    g32 = ops.flash_attn2_bwd(q, k, v, o, lse, do, scale, True, grad_f32=True)
    torch.cuda.synchronize()
    group = Hq // Hkv
    for b, hk in groups:
        print(f"  group b={b} kv head {hk}", flush=True)
        hs = slice(hk * group, (hk + 1) * group)
        qq, dd = host(q[b:b + 1, hs]), host(do[b:b + 1, hs])
        kk, vv = host(k[b:b + 1, hk:hk + 1]), host(v[b:b + 1, hk:hk + 1])
        oe, le = O.fa2_fwd(qq, kk, vv, scale, True)
        check_bf16(f"O[{b},{hk}]", host(o[b:b + 1, hs]), oe)
        assert np.abs(host(lse[b:b + 1, hs]) - le).max() <= 2e-2
        # the backward's inputs include O and LSE: give the oracle the same ones
        og, lg = host(o[b:b + 1, hs]), host(lse[b:b + 1, hs])
        want = O.fa2_bwd(qq, kk, vv, og, dd, lg, scale, True)
        got16 = (dq[b:b + 1, hs], dk[b:b + 1, hk:hk + 1], dv[b:b + 1, hk:hk + 1])
        got32 = (g32[0][b:b + 1, hs], g32[1][b:b + 1, hk:hk + 1], g32[2][b:b + 1, hk:hk + 1])
        for name, a, c, w in zip(("dQ", "dK", "dV"), got16, got32, want):
            check_bf16(f"{name}[{b},{hk}]", host(a), w)
            check_flat(f"{name}[{b},{hk}] (fp32)", host(c), w)
    assert torch.isfinite(dq.float()).all() and torch.isfinite(dk.float()).all()
    assert torch.isfinite(dv.float()).all()


def test_fa2_bf16_c3_full_size(cuda):
    """B8 H32 S4096 D128 causal, the headline shape: two whole heads."""
    _group_check(8, 32, 32, 4096, 128, seed=7, spike=False, groups=[(0, 0), (7, 31)])


@pytest.mark.parametrize("S", [16384, 8191])
def test_fa2_bf16_c5_long_gqa(cuda, S):
    """B1 Hq64 Hkv8 D128 causal, 1% of K rows x8; S = 16384 (each group's q
    heads split over 4 dK/dV workgroups, fp32 partials and their merge) and
    ragged 8191 (dK/dV in two wavefront groups per workgroup): one whole
    GQA group of 8 q heads."""
    _group_check(1, 64, 8, S, 128, seed=8, spike=True, groups=[(0, 5)])


@pytest.mark.parametrize("B,S,groups", [(2, 4096, [(1, 7)]), (16, 512, [(15, 3)]),
                                         (8, 1024, [(0, 0), (7, 5)])])
def test_fa2_bf16_gqa4_packed_group(cuda, B, S, groups):
    """Causal GQA groups of 4 (Hq32 Hkv8 D128), which run the GQA-packed
    forward and dQ: B2 S4096 (its dK/dV runs in two wavefront groups per
    workgroup), the Llama-3-8B prefill's B16 S512 and B8 S1024 (below 2048
    rows, all 512 dK/dV workgroups resident at once, heavy and light key
    blocks paired on each CU); whole groups, 1% of K rows x8."""
    _group_check(B, 32, 8, S, 128, seed=9 + S, spike=True, groups=groups)


@pytest.mark.parametrize("B,Hq,Hkv,S,D,groups", [(8, 32, 8, 1024, 64, [(3, 2)]),
                                                 (2, 32, 32, 1024, 128, [(1, 31), (0, 0)])])
def test_fa2_bf16_dkdv_cu_pairs(cuda, B, Hq, Hkv, S, D, groups):
    """Causal shapes whose 512 dK/dV workgroups are all resident at once, so
    the kernel pairs heavy and light key blocks on each CU: GQA 4 at D = 64
    and MHA at D = 128; whole groups against the oracle."""
    _group_check(B, Hq, Hkv, S, D, seed=11 + S + D, spike=True, groups=groups)

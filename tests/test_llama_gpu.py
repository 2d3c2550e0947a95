"""GPU parity of the Llama path: the fused QKV split + RoPE + cache write,
decode attention over a KV cache, one LlamaBlock against an oracle
composition of the reference's ops, and greedy generation with the KV cache
against the reference's recompute-every-step method."""
import dataclasses
import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from teenyformers_amd import llama, ops

pytestmark = pytest.mark.gpu


def f32_ln(x):
    return float(np.log(np.float32(x)).astype(np.float32))


def host(t):
    return t.float().cpu().numpy()


def rel_l2(a, b):
    return float(np.linalg.norm((a - b).ravel()) / np.linalg.norm(b.ravel()))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_qkv_rope_split(cuda, dtype):
    B, S, Hq, Hkv, D, pos0, L, base = 2, 37, 8, 2, 64, 5, 64, 5e5
    g = torch.Generator(device="cuda").manual_seed(3)
    qkv = torch.randn((B, S, (Hq + 2 * Hkv) * D), generator=g, device="cuda").to(dtype)
    q = torch.empty((B, Hq, S, D), dtype=dtype, device="cuda")
    kc = torch.zeros((B, Hkv, L, D), dtype=dtype, device="cuda")
    vc = torch.zeros_like(kc)
    ops.qkv_rope_split(qkv, q, kc, vc, pos0, Hq, Hkv, base)
    x = host(qkv).reshape(B, S, Hq + 2 * Hkv, D).transpose(0, 2, 1, 3)  # [B, H, S, D]

    def rope_at(t):  # oracle RoPE at positions pos0.. (pad rows in front)
        pad = np.zeros(t.shape[:2] + (pos0,) + t.shape[3:], np.float32)
        return O.rope(np.concatenate([pad, t], axis=2), f32_ln(base))[:, :, pos0:]

    want_q = rope_at(x[:, :Hq])
    want_k = rope_at(x[:, Hq:Hq + Hkv])
    tol = 1e-5 if dtype == torch.float32 else 2.0 ** -7
    assert np.abs(host(q) - want_q).max() <= tol * max(1.0, np.abs(want_q).max())
    assert np.abs(host(kc[:, :, pos0:pos0 + S]) - want_k).max() <= tol * max(1.0, np.abs(want_k).max())
    assert torch.equal(vc[:, :, pos0:pos0 + S],
                       qkv.view(B, S, Hq + 2 * Hkv, D)[:, :, Hq + Hkv:].transpose(1, 2))
    assert not kc[:, :, :pos0].any() and not kc[:, :, pos0 + S:].any()  # nothing else written


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n_keys,L,D,Hq,Hkv", [
    (1, 768, 64, 4, 4), (300, 768, 128, 32, 8), (700, 768, 64, 8, 1),
    # cache length off the 32-key tile: the last tile re-reads the last row
    (757, 757, 128, 16, 1),
    # many key splits, the last holding one key
    (2049, 4100, 128, 8, 8), (5000, 5000, 64, 32, 2)])
def test_decode_attention(cuda, dtype, n_keys, L, D, Hq, Hkv):
    B = 3
    g = torch.Generator(device="cuda").manual_seed(4)
    q = torch.randn((B, Hq, D), generator=g, device="cuda").to(dtype)
    kc = torch.randn((B, Hkv, L, D), generator=g, device="cuda").to(dtype)
    vc = torch.randn((B, Hkv, L, D), generator=g, device="cuda").to(dtype)
    scale = 1.0 / math.sqrt(D)
    o = ops.decode_attention(q, kc, vc, n_keys, scale)
    # the newest query sees every cached key: the non-causal forward with one row
    want, _ = O.fa2_fwd(host(q)[:, :, None], host(kc[:, :, :n_keys]), host(vc[:, :, :n_keys]),
                        scale, causal=False)
    want = want[:, :, 0]
    if dtype == torch.float32:
        assert np.abs(host(o) - want).max() <= 1e-5
    else:
        assert rel_l2(host(o), want) <= 5e-3 and np.abs(host(o) - want).max() <= 2e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n_keys,L,D,Hq,Hkv", [(300, 768, 128, 32, 8), (45, 64, 64, 8, 2),
                                               (1001, 1100, 128, 16, 1)])
def test_decode_attention_ignores_rows_past_n_keys(cuda, dtype, n_keys, L, D, Hq, Hkv):
    """Cache rows at or past n_keys (never written, or stale) may hold
    anything, NaN included: the output depends only on rows below n_keys.
    Host-position and device-position calls, n_keys off the 32-key tile; and
    the device-position call attends min(n_past + 1, max_keys) rows."""
    B = 2
    g = torch.Generator(device="cuda").manual_seed(5)
    q = torch.randn((B, Hq, D), generator=g, device="cuda").to(dtype)
    kc = torch.randn((B, Hkv, L, D), generator=g, device="cuda").to(dtype)
    vc = torch.randn((B, Hkv, L, D), generator=g, device="cuda").to(dtype)
    kc[:, :, n_keys:] = float("nan")
    vc[:, :, n_keys:] = float("nan")
    scale = 1.0 / math.sqrt(D)
    want, _ = O.fa2_fwd(host(q)[:, :, None], host(kc[:, :, :n_keys]), host(vc[:, :, :n_keys]),
                        scale, causal=False)
    want = want[:, :, 0]
    pdev = torch.tensor([n_keys - 1], dtype=torch.int32, device="cuda")
    for o in (ops.decode_attention(q, kc, vc, n_keys, scale),
              ops.decode_attention(q, kc, vc, L, scale, n_past=pdev)):
        got = host(o)
        assert np.isfinite(got).all()
        if dtype == torch.float32:
            assert np.abs(got - want).max() <= 1e-5
        else:
            assert rel_l2(got, want) <= 5e-3 and np.abs(got - want).max() <= 2e-2
    # max_keys below n_past + 1 caps the rows attended
    cap = n_keys - 7
    o_cap = ops.decode_attention(q, kc, vc, cap, scale, n_past=pdev)
    assert torch.equal(o_cap, ops.decode_attention(q, kc, vc, cap, scale))


def _oracle_block(cfg, w, x, r0=0):
    """One LlamaBlock from the oracle's restated ops + float32 numpy GEMMs:
    the output rows r0.. of x [B, S, d] (their queries attend every key up
    to their own position, q_offset r0)."""
    B, S, d = x.shape
    Hq, Hkv, D = cfg.n_heads, cfg.n_kv_heads(), cfg.head_dim()
    W = {k: host(v) for k, v in w.items() if k.startswith("model.layers.0.")}
    p = "model.layers.0."
    x2d = x.reshape(B * S, d)
    n1, _ = O.rmsnorm_fwd(x2d, W[p + "input_layernorm.weight"], cfg.eps)
    qkv = (n1 @ W[p + "self_attn.qkv_proj.weight"].T).reshape(B, S, Hq + 2 * Hkv, D)
    q = np.ascontiguousarray(qkv[:, r0:, :Hq].transpose(0, 2, 1, 3))
    k = np.ascontiguousarray(qkv[:, :, Hq:Hq + Hkv].transpose(0, 2, 1, 3))
    v = np.ascontiguousarray(qkv[:, :, Hq + Hkv:].transpose(0, 2, 1, 3))
    lnb = f32_ln(cfg.rope_base)
    o, _ = O.fa2_fwd(O.rope(q, lnb, pos0=r0), O.rope(k, lnb), v, cfg.softmax_scale(),
                     causal=True, q_offset=r0)
    S, x2d = S - r0, x[:, r0:].reshape(B * (S - r0), d)
    attn = O.transpose_heads(o, B, S, Hq, D, merge=True).reshape(B * S, Hq * D)
    x2 = x2d + attn @ W[p + "self_attn.o_proj.weight"].T
    n2, _ = O.rmsnorm_fwd(x2, W[p + "post_attention_layernorm.weight"], cfg.eps)
    f = O.swiglu_fwd(n2 @ W[p + "mlp.gate_up_proj.weight"].T) @ W[p + "mlp.down_proj.weight"].T
    return (x2 + f).reshape(B, S, d)


def test_block_f32_matches_oracle(cuda):
    cfg = llama.LlamaConfig(d_model=64, n_heads=4, n_layers=1, vocab_size=64, eps=1e-5,
                            rope_base=5e5, intermediate_size=128, n_kv_heads_=2)
    w = llama.init_weights(cfg, dtype=torch.float32, std=0.2, seed=5)
    x = torch.randn((2, 37, 64), generator=torch.Generator(device="cuda").manual_seed(6),
                    device="cuda")
    got = host(llama.block_forward(cfg, w, x))
    want = _oracle_block(cfg, w, host(x))
    assert np.abs(got - want).max() <= 1e-4 * max(1.0, np.abs(want).max())


C2 = dict(d_model=2048, n_heads=32, n_layers=1, vocab_size=32, eps=1e-5, rope_base=5e5,
          intermediate_size=8192, n_kv_heads_=8)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_block_c2_shape_sampled(cuda, dtype):
    """B4 S2048 d2048, Hq32 Hkv8 D64, F8192, eps 1e-5, theta 5e5, causal.
    Causal rows 0..R-1 depend only on rows 0..R-1, so the oracle checks the
    first 64 rows of two sequences at full width, and rows 1984..2047 of
    each (their attention over all 2048 keys, the GQA-packed kernel's last
    query blocks; the oracle forms K/V of the whole sequence and only these
    rows' queries).
    fp32 (the reference's precision): max abs <= 1e-4 of the output scale.
    bf16: rel-L2 <= 5e-3 and max abs <= 5e-2.  The composed block runs four
    bf16 GEMMs (K = 2048 and 8192) and stores its residual stream in bf16
    twice; attention and FFN each add O(1) to it, so the elementwise error is
    noise of sigma ~ 8e-3 whose maximum over the 2.6e5 checked elements sits
    near 4.5 sigma."""
    cfg = llama.LlamaConfig(**C2)
    w = llama.init_weights(cfg, dtype=dtype, std=0.02, seed=7)
    x = torch.randn((4, 2048, 2048), generator=torch.Generator(device="cuda").manual_seed(8),
                    device="cuda").to(dtype)
    got = llama.block_forward(cfg, w, x)
    torch.cuda.synchronize()
    for b, r0 in ((0, 0), (3, 0), (0, 1984), (3, 1984)):
        if r0 == 0:
            want = _oracle_block(cfg, w, host(x[b:b + 1, :64]))
        else:
            want = _oracle_block(cfg, w, host(x[b:b + 1]), r0)
        g = host(got[b:b + 1, r0:r0 + 64])
        err = np.abs(g - want)
        msg = f"b={b} rows {r0}.. rel-L2 {rel_l2(g, want):.3e} max abs {err.max():.3e}"
        print(f"block C2 {dtype}: {msg}", flush=True)
        if dtype == torch.float32:
            assert err.max() <= 1e-4 * max(1.0, np.abs(want).max()), msg
        else:
            assert rel_l2(g, want) <= 5e-3 and err.max() <= 5e-2, msg


@pytest.mark.parametrize("n_kv", [2, 4])
def test_generate_cached_equals_recompute(cuda, n_kv):
    """Greedy ids with the KV cache == ids from recomputing the whole sequence
    every step (the reference's method), fp32."""
    cfg = llama.LlamaConfig(d_model=128, n_heads=4, n_layers=2, vocab_size=512, eps=1e-5,
                            rope_base=1e4, intermediate_size=256, n_kv_heads_=n_kv)
    w = llama.init_weights(cfg, dtype=torch.float32, std=0.2, seed=9)
    model = llama.Llama(cfg, w)
    prompt = torch.randint(0, 512, (2, 12), generator=torch.Generator(device="cuda").manual_seed(10),
                           device="cuda")
    cached = model.generate(prompt, 10)
    recomputed = model.generate_recompute(prompt, 10)
    assert torch.equal(cached, recomputed), (cached, recomputed)
    # and the prefill logits equal the all-position forward's last row
    full = model.forward(prompt)
    _, last = model.prefill(prompt, 32)
    assert torch.allclose(full[:, -1], last, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_argmax_rows(cuda, dtype):
    """Last index of the row maximum (the reference's Iterator::max_by), NaN
    counting as the maximum."""
    g = torch.Generator(device="cuda").manual_seed(21)
    x = torch.randn((16, 128256), generator=g, device="cuda").to(dtype)
    x[3, 7] = x[3, 90000] = 1e4  # tie: the last index wins
    x[5, :] = 0.0                # all equal: the last index
    x[9, 123] = float("nan")     # NaN is the maximum
    x[11, :] = float("-inf")     # all -inf: the last index
    x[13, 5] = x[13, 70000] = float("nan")  # two NaNs, in different load batches: the last
    got = ops.argmax_rows(x)
    n = x.shape[1]
    # torch.argmax keeps the first maximum (and the first NaN): flip the row
    assert torch.equal(got, n - 1 - torch.argmax(x.flip(-1), dim=-1))
    assert got[3] == 90000 and got[5] == n - 1 and got[9] == 123 and got[11] == n - 1
    assert got[13] == 70000
    # a row whose length is not a multiple of the vector width
    y = x[:, :1001].contiguous()
    assert torch.equal(ops.argmax_rows(y), 1000 - torch.argmax(y.flip(-1), dim=-1))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_device_position_variants(cuda, dtype):
    """qkv_rope_split / decode_attention with the position in device memory
    equal the host-position calls; a position past the cache writes nothing."""
    B, Hq, Hkv, D, L, base = 2, 8, 2, 64, 300, 5e5
    g = torch.Generator(device="cuda").manual_seed(22)
    qkv = torch.randn((B, 1, (Hq + 2 * Hkv) * D), generator=g, device="cuda").to(dtype)
    kc0 = torch.randn((B, Hkv, L, D), generator=g, device="cuda").to(dtype)
    vc0 = torch.randn((B, Hkv, L, D), generator=g, device="cuda").to(dtype)
    for pos in (0, 17, 299):
        q_h, q_d = (torch.empty((B, Hq, 1, D), dtype=dtype, device="cuda") for _ in range(2))
        kh, vh, kd, vd = kc0.clone(), vc0.clone(), kc0.clone(), vc0.clone()
        ops.qkv_rope_split(qkv, q_h, kh, vh, pos, Hq, Hkv, base)
        pdev = torch.tensor([pos], dtype=torch.int32, device="cuda")
        ops.qkv_rope_split(qkv, q_d, kd, vd, pdev, Hq, Hkv, base)
        assert torch.equal(q_h, q_d) and torch.equal(kh, kd) and torch.equal(vh, vd)
        o_h = ops.decode_attention(q_h.view(B, Hq, D), kh, vh, pos + 1)
        o_d = ops.decode_attention(q_d.view(B, Hq, D), kd, vd, L, n_past=pdev)
        assert torch.equal(o_h, o_d)
    # past the cache: q is formed, the cache is untouched
    kd, vd = kc0.clone(), vc0.clone()
    q_d = torch.empty((B, Hq, 1, D), dtype=dtype, device="cuda")
    ops.qkv_rope_split(qkv, q_d, kd, vd, torch.tensor([L], dtype=torch.int32, device="cuda"),
                       Hq, Hkv, base)
    torch.cuda.synchronize()
    assert torch.equal(kd, kc0) and torch.equal(vd, vc0)


@pytest.mark.parametrize("B,Hq,Hkv,D,L", [
    (4, 32, 8, 128, 640),   # the Llama-3-8B decode shape
    (3, 8, 1, 64, 300),     # 8 q heads on one kv head, cache off the 32-key tile
    (2, 32, 1, 128, 1000),  # a 32-head group: every row of the score product
])
def test_decode_qkv_attention_fused(cuda, B, Hq, Hkv, D, L):
    """The one-launch decode step (QKV split + RoPE + cache write +
    attention) writes the same cache rows as teeny_qkv_rope_split_partials_dev
    (bit for bit) and its output matches the oracle's attention of that q
    over the cache rows 0 .. pos (row pos being the new k, v); rows past pos
    hold NaN and are not read; a position past the cache writes nothing."""
    rng = np.random.default_rng(B * 131 + Hq + D + L)
    d = 512
    n = (Hq + 2 * Hkv) * D
    x = _bf16_dev(rng.standard_normal((B, 1, d)).astype(np.float32))
    wq = _bf16_dev((0.05 * rng.standard_normal((n, d))).astype(np.float32))
    pq = ops.linear_split(x, wq, 128)
    assert pq.n == 4
    kc0 = _bf16_dev(rng.standard_normal((B, Hkv, L, D)).astype(np.float32))
    vc0 = _bf16_dev(rng.standard_normal((B, Hkv, L, D)).astype(np.float32))
    scale = 1.0 / math.sqrt(D)
    # row pos at a tile's first and last key, in a wavefront's first and a
    # later tile, the last cache row, and past the cache
    for pos in (0, 31, 32, 37 % L, 300 % L, L - 1, L):
        kc, vc = kc0.clone(), vc0.clone()
        kc[:, :, pos + 1:] = float("nan")
        vc[:, :, pos + 1:] = float("nan")
        pdev = torch.tensor([pos], dtype=torch.int32, device="cuda")
        q = torch.empty((B, Hq, 1, D), dtype=torch.bfloat16, device="cuda")
        k1, v1, k2, v2 = kc.clone(), vc.clone(), kc.clone(), vc.clone()
        ops.qkv_rope_split(pq, q, k1, v1, pdev, Hq, Hkv, 5e5)
        o = ops.decode_qkv_attention(pq, k2, v2, pdev, Hq, Hkv, 5e5, scale)
        torch.cuda.synchronize()
        print(f"decode_qkv: B{B} Hq{Hq} Hkv{Hkv} D{D} L{L} pos {pos}", flush=True)
        assert torch.equal(k1.view(torch.int16), k2.view(torch.int16))
        assert torch.equal(v1.view(torch.int16), v2.view(torch.int16))
        n_keys = min(pos + 1, L)
        want, _ = O.fa2_fwd(host(q), host(k1[:, :, :n_keys]), host(v1[:, :, :n_keys]), scale,
                            causal=False)
        got = host(o)
        assert np.isfinite(got).all()
        assert rel_l2(got, want[:, :, 0]) <= 5e-3 and np.abs(got - want[:, :, 0]).max() <= 2e-2


@pytest.mark.parametrize("dtype,batch", [(torch.float32, 3), (torch.bfloat16, 3),
                                         (torch.bfloat16, 20), (torch.float32, 20)])
def test_generate_graph_equals_eager(cuda, dtype, batch):
    """Greedy ids from the decode step captured in a HIP graph and replayed
    (8 replays, eager work between them) == ids from the eager decode loop.
    With 3 sequences the bf16 step runs the weight-streaming decode kernels;
    with 20 (more than 16 rows) its products run the library's own GEMM both
    eagerly and captured (a captured teeny_linear_bf16 never runs hipBLASLt),
    and the fp32 step runs teeny_linear_f32, whose capture runs the own fp32
    GEMM: the eager loop follows the same rule, so the bits agree."""
    cfg = llama.LlamaConfig(d_model=256, n_heads=4, n_layers=2, vocab_size=512, eps=1e-5,
                            rope_base=1e4, intermediate_size=512, n_kv_heads_=2)
    w = llama.init_weights(cfg, dtype=dtype, std=0.2, seed=23)
    model = llama.Llama(cfg, w)
    prompt = torch.randint(0, 512, (batch, 9),
                           generator=torch.Generator(device="cuda").manual_seed(24),
                           device="cuda")
    eager = model.generate(prompt, 10)
    graph = model.generate_graph(prompt, 10)
    assert torch.equal(eager, graph), (eager, graph)


def test_generate_stream_layout_equals_row_major(cuda):
    """Greedy ids of the graph-replayed decode with the weights in the
    streaming layout (ops.StreamWeight) == the eager decode from the
    row-major weights: the layout changes only the order of the loads."""
    cfg = llama.LlamaConfig(d_model=256, n_heads=4, n_layers=2, vocab_size=512, eps=1e-5,
                            rope_base=1e4, intermediate_size=512, n_kv_heads_=2)
    w = llama.init_weights(cfg, dtype=torch.bfloat16, std=0.2, seed=29)
    prompt = torch.randint(0, 512, (5, 9), generator=torch.Generator(device="cuda").manual_seed(30),
                           device="cuda")
    eager = llama.Llama(cfg, w).generate(prompt, 10)
    model = llama.Llama(cfg, w).stream_layout()
    assert len(model.sw) == 1 + 4 * cfg.n_layers
    graph = model.generate_graph(prompt, 10)
    assert torch.equal(eager, graph), (eager, graph)


def _bf16_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda", torch.bfloat16)


@pytest.mark.parametrize("N,K", [(16, 128), (48, 640), (4096, 4224)])
def test_stream_layout(cuda, N, K):
    """teeny_linear_stream_layout_bf16 against its definition:
    w_s[nb][ks][q][g][r][e] = W[16 nb + r][128 ks + 32 g + 8 q + e]."""
    w = torch.randn(N, K, device="cuda").to(torch.bfloat16)
    got = ops.StreamWeight(w).s.view(torch.int16).cpu().numpy()
    want = (w.view(torch.int16).cpu().numpy().reshape(N // 16, 16, K // 128, 4, 4, 8)
            .transpose(0, 2, 4, 3, 1, 5).reshape(N, K))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("M,N,K,k_split", [
    (1, 128, 128, None), (5, 256, 640, None),    # partial 512-wide chunks
    (16, 4096, 4096, None), (16, 6144, 4096, 896), (16, 4096, 14336, 1792),
    (7, 128, 4224, 384), (16, 1024, 4096, 4096)])
def test_linear_stream_layout_bit_exact(cuda, M, N, K, k_split):
    """The decode linears reading the streaming layout give the same bits
    as the row-major kernels: the product (teeny_linear_sl_bf16), the
    K-split slabs (teeny_linear_partials_sl_bf16) and, on [N, K] read as a
    fused [2F, K] gate_up weight, SwiGLU (teeny_linear_swiglu_sl_bf16)."""
    g = torch.Generator(device="cuda").manual_seed(M * 131 + N + K)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    w = (0.02 * torch.randn(N, K, device="cuda", generator=g)).to(torch.bfloat16)
    sw = ops.StreamWeight(w)
    assert torch.equal(ops.linear(x, sw), ops.linear(x, w))
    p_sl, p_rm = ops.linear_split(x, sw, k_split), ops.linear_split(x, w, k_split)
    assert p_sl.n == p_rm.n and torch.equal(p_sl.slabs, p_rm.slabs)
    if N % 128 == 0:  # F = N / 2, a multiple of 64
        assert torch.equal(ops.linear_swiglu(x, sw), ops.linear_swiglu(x, w))
    # more than 16 rows: the row-major weight (the GEMM), same as without it
    x20 = torch.randn(20, K, device="cuda", generator=g).to(torch.bfloat16)
    assert torch.equal(ops.linear(x20, sw), ops.linear(x20, w))


@pytest.mark.parametrize("M,N,K", [
    (1, 128, 128), (5, 256, 256),       # one partial 512-wide x chunk
    (16, 4096, 4096), (16, 128, 14336), # decode shapes: o_proj, down
    (3, 1024, 640), (16, 128, 4224)])   # a last chunk of one 128-wide step
def test_linear_skinny(cuda, M, N, K):
    """Decode-step linear against float64 matmul of the same bf16 operands:
    within one bf16 rounding of the output (summation order differs)."""
    rng = np.random.default_rng(M * 7919 + N + K)
    x = O.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    w = O.bf16_round((0.02 * rng.standard_normal((N, K))).astype(np.float32))
    y = ops.linear(_bf16_dev(x), _bf16_dev(w))
    want = x.astype(np.float64) @ w.astype(np.float64).T
    err = np.abs(host(y) - want)
    assert np.all(err <= np.abs(want) * 2.0 ** -8 + 1e-4 * np.abs(want).max()), err.max()
    # deterministic: the same bits on a second call
    assert torch.equal(y, ops.linear(_bf16_dev(x), _bf16_dev(w)))
    # the K-split form: slabs sum to the same product
    part = ops.linear_split(_bf16_dev(x), _bf16_dev(w))
    slabs = part.slabs.cpu().numpy()
    tot = slabs.sum(0, dtype=np.float64)
    assert np.all(np.abs(tot - want) <= np.abs(want) * 2.0 ** -16 + 1e-5 * np.abs(want).max())


def _seq_sum_bf16(slabs):
    """Slab-order fp32 sum rounded to bf16, as the consumers add them."""
    acc = np.zeros(slabs.shape[1:], np.float32)
    for s in slabs:
        acc = (acc + s).astype(np.float32)
    return O.bf16_round(acc)


@pytest.mark.parametrize("d,k_split", [
    (2048, None), (2048, 384), (2048, 128),  # 16, 6 (a last group of 6) and 16 slabs
    (4096, 640), (8192, 1152)])              # 7 and 8 slabs of 2 and 4 chunks per thread
def test_partials_consumers_bit_exact(cuda, d, k_split):
    """The residual-add norm and the QKV split read K-split slabs exactly as
    they read the stored bf16 product."""
    rng = np.random.default_rng(11 + d + (k_split or 0))
    B, Hq, Hkv, D, L = 4, 8, 2, 64, 64
    n = (Hq + 2 * Hkv) * D
    x = _bf16_dev(rng.standard_normal((B, d)).astype(np.float32))
    wq = _bf16_dev((0.02 * rng.standard_normal((n, d))).astype(np.float32))
    wo = _bf16_dev((0.02 * rng.standard_normal((d, d))).astype(np.float32))
    res = _bf16_dev(rng.standard_normal((B, d)).astype(np.float32))
    gamma = _bf16_dev((1 + 0.1 * rng.standard_normal(d)).astype(np.float32))
    po = ops.linear_split(x, wo, k_split)
    assert po.n > 1
    a = _bf16_dev(_seq_sum_bf16(po.slabs.cpu().numpy()))
    y1, h1, r1 = ops.fused_add_rmsnorm(po, res, gamma, 1e-5)
    y2, h2, r2 = ops.fused_add_rmsnorm(a, res, gamma, 1e-5)
    assert torch.equal(y1, y2) and torch.equal(h1, h2) and torch.equal(r1, r2)
    pq = ops.linear_split(x.view(B, 1, d), wq, k_split)
    qkv = _bf16_dev(_seq_sum_bf16(pq.slabs.cpu().numpy())).view(B, 1, n)
    pos = torch.tensor([17], dtype=torch.int32, device="cuda")
    outs = []
    for src in (pq, qkv):
        q = torch.zeros((B, Hq, 1, D), dtype=torch.bfloat16, device="cuda")
        kc = torch.zeros((B, Hkv, L, D), dtype=torch.bfloat16, device="cuda")
        vc = torch.zeros_like(kc)
        ops.qkv_rope_split(src, q, kc, vc, pos, Hq, Hkv, 5e5)
        outs.append((q, kc, vc))
    for t1, t2 in zip(*outs):
        assert torch.equal(t1, t2)


@pytest.mark.parametrize("M,F,K", [(16, 14336 // 8, 4096), (2, 64, 640)])
def test_linear_swiglu_skinny(cuda, M, F, K):
    """Fused gate_up product + SwiGLU against the unfused composition: the
    float64 product rounded to bf16, then the oracle's SwiGLU."""
    rng = np.random.default_rng(F + K)
    x = O.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    w = O.bf16_round((0.02 * rng.standard_normal((2 * F, K))).astype(np.float32))
    y = ops.linear_swiglu(_bf16_dev(x), _bf16_dev(w))
    z = O.bf16_round((x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32))
    want = O.bf16_round(O.swiglu_fwd(z))
    err = np.abs(host(y) - want)
    # one bf16 step of z can move silu(g) * u by a few output ulps
    assert np.all(err <= np.abs(want) * 2.0 ** -5 + 1e-3 * np.abs(want).max()), err.max()
    assert rel_l2(host(y), want) <= 5e-3


@pytest.mark.parametrize("M,F,K", [
    (8192, 1792, 4096),   # Llama-3-8B's MLP on 16 x 512 tokens, an eighth of its features
    (300, 96, 640),       # a ragged row tile; the feature tile three quarters full
    (17, 160, 128),       # one 64-deep K tile; a second feature tile of 32
    (5, 32, 192),         # few rows, F % 64 != 0: the GEMM, not the decode kernel
    (16, 448, 4096)])     # the decode kernel
def test_linear_swiglu_any_rows(cuda, M, F, K):
    """teeny_linear_swiglu_bf16 at any M gives the bits of the unfused
    composition with the same kernel (the decode kernel up to 16 rows, the
    library's own GEMM above, on the [2F, K] weight, then the SwiGLU kernel),
    and that composition is within the bf16 tolerance of the float64
    product; above 16 rows the linear entry point (hipBLASLt) is within one
    bf16 rounding of the own GEMM."""
    rng = np.random.default_rng(M + 3 * F + K)
    x = _bf16_dev(rng.standard_normal((M, K)).astype(np.float32))
    w = _bf16_dev((0.02 * rng.standard_normal((2 * F, K))).astype(np.float32))
    y = torch.empty((M, F), dtype=torch.bfloat16, device="cuda")
    call = lambda: ops.call("teeny_linear_swiglu_bf16", ops._p(x), ops._p(w), ops._p(y), M, F, K,
                            ops._stream())
    call()
    z = ops.linear(x, w) if (M <= 16 and F % 64 == 0 and K % 128 == 0) else ops.gemm_own(x, w)
    assert torch.equal(y, ops.swiglu(z))
    y1 = y.clone()
    call()
    assert torch.equal(y, y1)  # deterministic
    if M > 16:
        zl, zo = ops.linear(x, w).float(), z.float()
        assert torch.all((zl - zo).abs() <= zo.abs() * 2.0 ** -7 + 1e-6)
    if M * F <= 1 << 20:
        xh, wh = host(x).astype(np.float64), host(w).astype(np.float64)
        zh = O.bf16_round((xh @ wh.T).astype(np.float32))
        want = O.bf16_round(O.swiglu_fwd(zh))
        assert rel_l2(host(y), want) <= 5e-3

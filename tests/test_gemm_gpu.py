"""The prompt-size Linear behind sym_linear (reference src/layers/mod.rs:54-58,
y = x W^T with W [out, in]) through both entry points: the library's own
matrix-core GEMM (teeny_gemm_bf16, gemm_bf16.hip) and teeny_linear_bf16
(hipBLASLt above 16 rows, the own GEMM as its fallback), against float64
products of the same bf16 operands.  Bar: one bf16 rounding of the output
(|got - want| <= 2^-8 |want|, plus 1e-6 of the output scale for the fp32
summation order).  And the fp32 Linear (the reference's own precision):
teeny_linear_f32 (hipBLASLt) and teeny_gemm_f32 (gemm_f32.hip) against
float64 products within the fp32 dot-product error bound."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from teenyformers_amd import _lib, ops

pytestmark = pytest.mark.gpu


def _operands(M, N, K, seed):
    rng = np.random.default_rng(seed)
    x = O.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    w = O.bf16_round((0.02 * rng.standard_normal((N, K))).astype(np.float32))
    return x, w


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda", torch.bfloat16)


def _check(got, x, w):
    want = x.astype(np.float64) @ w.astype(np.float64).T
    err = np.abs(got - want)
    assert np.all(err <= np.abs(want) * 2.0 ** -8 + 1e-6 * np.abs(want).max()), err.max()


def _gemm(x, w, entry="teeny_linear_bf16"):
    """A bf16 product through the C ABI."""
    M, K = x.shape
    N = w.shape[0]
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    _lib.call(entry, ops._p(x), ops._p(w), ops._p(y), M, N, K, ops._stream())
    return y


ENTRIES = ["teeny_gemm_bf16", "teeny_linear_bf16"]


@pytest.mark.parametrize("entry", ENTRIES)
@pytest.mark.parametrize("M,N,K", [
    (17, 64, 64), (300, 192, 128), (1000, 320, 4160),  # ragged M, N off the 256 tile
    (5, 192, 256),                                      # few rows, N not a multiple of 128
    (257, 256, 512), (511, 768, 2048), (4096, 64, 64)])
def test_gemm_small(cuda, M, N, K, entry):
    x, w = _operands(M, N, K, seed=M + N + K)
    y = _gemm(_dev(x), _dev(w), entry)
    _check(y.float().cpu().numpy(), x, w)
    assert torch.equal(y, _gemm(_dev(x), _dev(w), entry))  # deterministic


@pytest.mark.parametrize("entry", ENTRIES)
@pytest.mark.parametrize("M,N,K", [
    (8192, 6144, 4096), (8192, 4096, 4096), (8192, 28672, 4096), (8192, 4096, 14336),  # 8B shape
    (8192, 3072, 2048), (8192, 2048, 2048), (8192, 16384, 2048), (8192, 2048, 8192),   # block
    (64, 128256, 4096)])                                                               # lm_head
def test_gemm_llama_shapes(cuda, M, N, K, entry):
    """The prompt GEMMs of the Llama-3-8B shape (B16 x 512 tokens) and of the
    Llama block (B4 x 2048), and the tied lm_head over 64 rows; rows from the
    first, a middle and the last 256-row tile are checked in full width."""
    x, w = _operands(M, N, K, seed=N + K)
    y = _gemm(_dev(x), _dev(w), entry)
    rows = sorted({*range(0, min(M, 64)), *range(max(0, M // 2 + 3), min(M, M // 2 + 35)),
                   *range(max(0, M - 64), M)})
    _check(y[rows].float().cpu().numpy(), x[rows], w)


def test_linear_wide_column_blocks(cuda):
    """The all-position lm_head (8192 x 128256 x 4096), for which hipBLASLt
    has no single algorithm: teeny_linear_bf16 runs it as column blocks of
    y.  Rows from three tiles against float64 products, and every output
    bit-equal to the own GEMM's (the same sums per output)."""
    M, N, K = 8192, 128256, 4096
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16)
    w = (0.02 * torch.randn((N, K), generator=g, device="cuda")).to(torch.bfloat16)
    y = _gemm(x, w)
    rows = [*range(0, 32), *range(M // 2 + 3, M // 2 + 35), *range(M - 32, M)]
    want = (x[rows].double() @ w.double().T)
    bar = want.abs() * 2.0 ** -8 + 1e-6 * want.abs().max()
    assert bool(((y[rows].double() - want).abs() <= bar).all())
    assert torch.equal(y, _gemm(x, w, "teeny_gemm_bf16"))


def test_gemm_linear_op(cuda):
    """ops.linear routes bf16 prompts to teeny_linear_bf16 (any leading shape)
    and still takes the decode kernels at 16 rows; ops.gemm_own is the own
    GEMM."""
    x, w = _operands(2 * 96, 512, 256, seed=3)
    y = ops.linear(_dev(x).view(2, 96, 256), _dev(w))
    _check(y.view(192, 512).float().cpu().numpy(), x, w)
    assert torch.equal(y.view(192, 512), _gemm(_dev(x), _dev(w)))
    assert torch.equal(ops.gemm_own(_dev(x), _dev(w)), _gemm(_dev(x), _dev(w), "teeny_gemm_bf16"))
    xs = _dev(x[:16])
    assert torch.equal(ops.linear(xs, _dev(w)), _gemm(xs, _dev(w)))


@pytest.mark.parametrize("seen_eagerly", [False, True])
def test_linear_under_graph_capture(cuda, seen_eagerly):
    """A prompt-size teeny_linear_bf16 inside a HIP graph capture always runs
    the own GEMM, whether or not the shape already ran eagerly (through
    hipBLASLt) before the capture: the graph's kernel does not depend on the
    call history.  The replays give the own GEMM's bits each time, with eager
    work between them."""
    M, N, K = (320, 384, 512) if seen_eagerly else (352, 448, 576)
    x, w = _operands(M, N, K, seed=9 + M)
    xd, wd = _dev(x), _dev(w)
    if seen_eagerly:
        _check(_gemm(xd, wd).float().cpu().numpy(), x, w)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        _lib.call("teeny_linear_bf16", ops._p(xd), ops._p(wd), ops._p(y), M, N, K,
                  torch.cuda.current_stream().cuda_stream)
    own = _gemm(xd, wd, "teeny_gemm_bf16")
    for _ in range(3):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, own)
        _check(_gemm(xd, wd).float().cpu().numpy(), x, w)  # eager: hipBLASLt


# ---------------------------------------------------------------------------
# fp32 Linear (the reference's precision): teeny_linear_f32 (hipBLASLt's fp32
# GEMM) and teeny_gemm_f32 (the library's own), against float64 products of
# the same operands.  Bar: the worst-case fp32 dot-product bound for any
# summation order, |err| <= 2 K u sum_k |x_k w_k| (u = 2^-24), and rel-L2
# within max(1e-6, u sqrt(K)) over the checked rows (a sequential fp32 sum
# of K random-sign terms has an rms relative error near u sqrt(K / 2)).
# ---------------------------------------------------------------------------
F32_ENTRIES = ["teeny_gemm_f32", "teeny_linear_f32"]


def _operands_f32(M, N, K, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((M, K)).astype(np.float32),
            (0.02 * rng.standard_normal((N, K))).astype(np.float32))


def _gemm_f32(x, w, entry):
    M, K = x.shape
    N = w.shape[0]
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    _lib.call(entry, ops._p(x), ops._p(w), ops._p(y), M, N, K, ops._stream())
    return y


def _check_f32(got, x, w):
    x64, w64 = x.astype(np.float64), w.astype(np.float64)
    want = x64 @ w64.T
    bound = 2.0 * x.shape[1] * 2.0 ** -24 * (np.abs(x64) @ np.abs(w64).T)
    err = np.abs(got - want)
    assert np.all(err <= bound), float((err / np.maximum(bound, 1e-30)).max())
    rel = float(np.linalg.norm(got - want) / np.linalg.norm(want))
    assert rel <= max(1e-6, 2.0 ** -24 * np.sqrt(x.shape[1])), rel
    return rel


@pytest.mark.parametrize("entry", F32_ENTRIES)
@pytest.mark.parametrize("M,N,K", [
    (1, 8, 4), (17, 70, 36), (300, 192, 128), (129, 129, 132),  # ragged M, N, K off the tiles
    (1000, 320, 4160), (5, 4096, 4096), (16, 128256, 512)])
def test_linear_f32_small(cuda, M, N, K, entry):
    x, w = _operands_f32(M, N, K, seed=M * 31 + N + K)
    xd, wd = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    y = _gemm_f32(xd, wd, entry)
    _check_f32(y.cpu().numpy(), x, w)
    assert torch.equal(y, _gemm_f32(xd, wd, entry))  # deterministic


@pytest.mark.parametrize("entry", F32_ENTRIES)
@pytest.mark.parametrize("M,N,K", [
    (8192, 6144, 4096), (8192, 4096, 14336),   # Llama-3-8B prompt: qkv, down
    (8192, 3072, 2048), (8192, 2048, 8192)])   # Llama block: qkv, down
def test_linear_f32_llama_shapes(cuda, M, N, K, entry):
    """fp32 prompt products at the Llama shapes; rows of the first, a middle
    and the last 128-row tile in full width."""
    x, w = _operands_f32(M, N, K, seed=N + K)
    y = _gemm_f32(torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), entry)
    rows = sorted({*range(0, 48), *range(M // 2 + 3, M // 2 + 35), *range(M - 48, M)})
    rel = _check_f32(y[rows].cpu().numpy(), x[rows], w)
    print(f"linear_f32 {entry} M{M} N{N} K{K}: rel-L2 {rel:.2e}", flush=True)


def test_linear_f32_op(cuda):
    """ops.linear routes fp32 products (no gradient) through teeny_linear_f32,
    not torch; ops.gemm_f32 is the own kernel."""
    x, w = _operands_f32(2 * 48, 320, 256, seed=5)
    xd, wd = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    y = ops.linear(xd.view(2, 48, 256), wd)
    assert torch.equal(y.view(96, 320), _gemm_f32(xd, wd, "teeny_linear_f32"))
    assert torch.equal(ops.gemm_f32(xd, wd), _gemm_f32(xd, wd, "teeny_gemm_f32"))
    _check_f32(y.view(96, 320).cpu().numpy(), x, w)


def test_linear_f32_under_graph_capture(cuda):
    """Under capture teeny_linear_f32 runs the own fp32 GEMM; replays give
    its bits each time."""
    M, N, K = 200, 96, 160
    x, w = _operands_f32(M, N, K, seed=12)
    xd, wd = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    _gemm_f32(xd, wd, "teeny_linear_f32")
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        _lib.call("teeny_linear_f32", ops._p(xd), ops._p(wd), ops._p(y), M, N, K,
                  torch.cuda.current_stream().cuda_stream)
    own = _gemm_f32(xd, wd, "teeny_gemm_f32")
    for _ in range(3):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, own)

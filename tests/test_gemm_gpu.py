"""The prompt-size Linear behind sym_linear (reference src/layers/mod.rs:54-58,
y = x W^T with W [out, in]) through both entry points: the library's own
matrix-core GEMM (teeny_gemm_bf16, gemm_bf16.hip) and teeny_linear_bf16
(hipBLASLt above 16 rows, the own GEMM as its fallback), against float64
products of the same bf16 operands.  Bar: one bf16 rounding of the output
(|got - want| <= 2^-8 |want|, plus 1e-6 of the output scale for the fp32
summation order)."""
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


def test_linear_under_graph_capture(cuda):
    """A prompt-size teeny_linear_bf16 first met inside a HIP graph capture
    runs the own GEMM (hipBLASLt's handle, plan and workspace are created
    outside captures only); the graph replays give the eager bits each
    time, with eager work between the replays."""
    M, N, K = 320, 384, 512
    x, w = _operands(M, N, K, seed=9)
    xd, wd = _dev(x), _dev(w)
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

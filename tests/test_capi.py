"""The C-ABI library without a GPU: it loads, exports every declared symbol,
and rejects bad arguments with the documented codes before launching
anything (validation runs before any HIP call)."""
import ctypes

import pytest

from teenyformers_amd import _lib

OK, NULLP, SHAPE, UNSUP, WS, VALUE, SCRATCH, NOT_INIT = 0, -1, -2, -3, -4, -7, -8, -9
GRAD_F32 = 0x100
F32, BF16 = 0, 1
NEG_INF = float("-inf")
P = 0x1000  # a non-null dummy pointer: never dereferenced by failing calls


@pytest.fixture(scope="module")
def L():
    return _lib.lib()


def test_exports_every_declared_symbol(L):
    declared = _lib.header_functions()
    assert len(declared) >= 20
    for name in declared:
        assert hasattr(L, name), name
    assert L.teeny_abi_version() == 1


def test_strerror(L):
    assert L.teeny_strerror(0).decode() == "ok"
    assert "workspace" in L.teeny_strerror(WS).decode()


def fwd(L, **kw):
    a = dict(q=P, k=P, v=P, o=P, l=P, nq=128, nk=128, scale=0.125, neg_inf=NEG_INF, b=1, hq=4,
             hkv=4, d=64, dtype=BF16)
    a.update(kw)
    return L.teeny_causal_flash_attn2_fwd(a["q"], a["k"], a["v"], a["o"], a["l"], a["nq"], a["nk"],
                                          a["scale"], a["neg_inf"], a["b"], a["hq"], a["hkv"],
                                          a["d"], a["dtype"], None)


def test_fa2_fwd_validation(L):
    assert fwd(L, q=None) == NULLP
    assert fwd(L, l=None) == NULLP
    assert fwd(L, nq=0) == SHAPE
    assert fwd(L, hq=6, hkv=4) == SHAPE  # Hq must be a multiple of Hkv
    assert fwd(L, d=96) == UNSUP
    assert fwd(L, d=32, dtype=BF16) == UNSUP  # bf16 built for 64/128
    assert fwd(L, dtype=7) == UNSUP
    assert fwd(L, neg_inf=-1e9) == VALUE  # the reference always passes -inf
    assert fwd(L, scale=float("nan")) == VALUE


def test_fa2_fwd_merged_validation(L):
    """The merged-heads forward validates like the forward and is bf16 only."""
    def m(causal=1, **kw):
        a = dict(q=P, nq=128, scale=0.125, dtype=BF16)
        a.update(kw)
        return L.teeny_flash_attn2_fwd_merged(a["q"], P, P, P, P, a["nq"], 128, a["scale"],
                                              NEG_INF, 1, 4, 4, 64, a["dtype"], causal, None)
    for c in (0, 1):
        assert m(c, dtype=F32) == UNSUP
        assert m(c, q=None) == NULLP
        assert m(c, nq=0) == SHAPE
        assert m(c, scale=0.0) == VALUE


def test_fa2_fwd_qkv_and_rope_table_validation(L):
    """The attention from the fused QKV projection validates like the
    forward, is bf16 only and needs a 16-byte aligned (cos, sin) table."""
    def f(**kw):
        a = dict(qkv=P, cs=P, nq=128, dtype=BF16, scale=0.125, d=64)
        a.update(kw)
        return L.teeny_flash_attn2_fwd_qkv(a["qkv"], a["cs"], P, P, P, P, a["nq"], 128, a["scale"],
                                           NEG_INF, 1, 4, 2, a["d"], a["dtype"], 1, None)
    assert f(dtype=F32) == UNSUP
    assert f(cs=None) == NULLP
    assert f(cs=P + 8) == VALUE
    assert f(qkv=None) == NULLP
    assert f(nq=0) == SHAPE
    assert f(d=96) == UNSUP
    assert f(scale=0.0) == VALUE
    assert f(nq=1 << 22, d=128) == SHAPE  # B*S*(Hq+2Hkv)*D past the 32-bit element range
    assert L.teeny_rope_table(None, 16, 64, 9.2, None) == NULLP
    assert L.teeny_rope_table(P, 0, 64, 9.2, None) == SHAPE
    assert L.teeny_rope_table(P, 16, 64, 9.2, None) == SHAPE  # positions in blocks of 32
    assert L.teeny_rope_table(P, 32, 40, 9.2, None) == SHAPE  # head_dim a multiple of 16
    assert L.teeny_rope_table(P, 32, 64, float("inf"), None) == VALUE


def test_fa2_scale_domain(L):
    """bf16 kernels fold the scale into the exponent after masking raw
    scores to -inf: scale must be > 0 there (0 or negative would turn masked
    scores into NaN or +inf)."""
    assert fwd(L, scale=0.0) == VALUE
    assert fwd(L, scale=-0.125) == VALUE
    assert fwd(L, scale=float("inf")) == VALUE
    ws = L.teeny_flash_attn2_bwd_workspace_bytes(128, 1, 4, 64, BF16)
    rc = L.teeny_causal_flash_attn2_bwd(P, P, P, P, P, P, P, P, P, 128, 128, 0.0, 1, 4, 4, 64,
                                        BF16, P, ws, None)
    assert rc == VALUE
    rc = L.teeny_decode_attention(P, P, P, P, 1, 4, 4, 10, 16, 64, -1.0, BF16, P, 1 << 20, None)
    assert rc == VALUE


def test_fa2_grad_f32_flag(L):
    """TEENY_GRAD_F32 changes the gradients' type, not the workspace."""
    for args in ((4096, 8, 32, 128), (300, 2, 8, 128), (128, 1, 4, 64)):
        assert L.teeny_flash_attn2_bwd_workspace_bytes(*args, BF16 | GRAD_F32) == \
            L.teeny_flash_attn2_bwd_workspace_bytes(*args, BF16)
    f = L.teeny_flash_attn2_bwd_workspace_bytes_gqa
    assert f(16384, 16384, 1, 64, 8, 128, BF16 | GRAD_F32) == \
        f(16384, 16384, 1, 64, 8, 128, BF16)
    # validation still applies to the flagged dtype
    rc = L.teeny_causal_flash_attn2_bwd(P, P, P, P, P, P, P, P, P, 128, 128, 0.125, 1, 4, 4, 32,
                                        BF16 | GRAD_F32, P, 1 << 20, None)
    assert rc == UNSUP


def test_noalloc_bwd_refuses_beyond_scratch(L):
    """The no-allocation backward's static array is 16 MiB per device;
    problems whose workspace exceeds it are refused before anything runs."""
    assert L.teeny_scratch_bytes() == 16 << 20
    # B8 Hq32 S4096 D128 needs 8 MiB: within; B8 Hq32 S16384 needs 32 MiB
    assert L.teeny_flash_attn2_bwd_workspace_bytes(4096, 8, 32, 128, BF16) <= 16 << 20
    assert L.teeny_flash_attn2_bwd_workspace_bytes(16384, 8, 32, 128, BF16) > 16 << 20
    rc = L.teeny_causal_flash_attn2_bwd_noalloc(P, P, P, P, P, P, P, P, P, 16384, 16384, 0.088,
                                                8, 32, 32, 128, BF16, None)
    assert rc == SCRATCH
    assert "scratch" in L.teeny_strerror(SCRATCH).decode()


def test_fa2_bwd_workspace_gqa(L):
    """The larger workspace that allows the dK/dV head split: only for bf16
    GQA with an even group, 12288+ query rows and few key blocks (at most
    four 128-key blocks x batch x kv heads per CU of a 256-CU device without
    a GPU to ask): fp32 dK and dV partials for 4 splits (2 when 4 does not
    divide the group) on top of the base workspace."""
    f = L.teeny_flash_attn2_bwd_workspace_bytes_gqa
    base = L.teeny_flash_attn2_bwd_workspace_bytes
    # B1 Hq64 Hkv8 S16384: 128 blocks x 8 kv heads = 1024 workgroups, split 4
    assert f(16384, 16384, 1, 64, 8, 128, BF16) == base(16384, 1, 64, 128, BF16) + \
        2 * 4 * 8 * 16384 * 128 * 4
    # group of 2: split 2 (the shape the no-allocation test runs)
    assert f(12288, 12288, 1, 2, 1, 64, BF16) == base(12288, 1, 2, 64, BF16) + \
        2 * 2 * 1 * 12288 * 64 * 4
    # 2048-12287 rows (two wavefront groups, no partials), short walks, MHA,
    # odd groups, many key blocks, fp32: nothing to split
    for args in ((8191, 8191, 1, 64, 8, 128), (4096, 4096, 2, 32, 8, 128),
                 (1024, 1024, 4, 32, 8, 128), (512, 512, 16, 32, 8, 128),
                 (16384, 16384, 1, 32, 32, 128), (16384, 16384, 1, 24, 8, 128),
                 (16384, 16384, 2, 64, 8, 128)):
        Sq, Sk, B, Hq, Hkv, D = args
        assert f(*args, BF16) == base(Sq, B, Hq, D, BF16), args
    assert f(128, 128, 1, 4, 2, 64, F32) == base(128, 1, 4, 64, F32)
    assert f(16384, 16384, 1, 64, 8, 128, F32) == base(16384, 1, 64, 128, F32)
    assert f(128, 128, 1, 6, 4, 64, BF16) == 0  # Hq % Hkv != 0
    assert f(0, 128, 1, 4, 2, 64, BF16) == 0


def test_fa2_bwd_workspace(L):
    need = L.teeny_flash_attn2_bwd_workspace_bytes(4096, 8, 32, 128, BF16)
    rows = 8 * 32 * 4096
    assert need >= rows * 4  # Delta
    assert L.teeny_flash_attn2_bwd_workspace_bytes(128, 1, 4, 64, F32) >= 4 * 128 * 4
    small = L.teeny_flash_attn2_bwd_workspace_bytes(128, 1, 4, 64, BF16)
    rc = L.teeny_causal_flash_attn2_bwd(P, P, P, P, P, P, P, P, P, 128, 128, 0.125, 1, 4, 4, 64,
                                        BF16, P, small - 1, None)
    assert rc == WS
    rc = L.teeny_causal_flash_attn2_bwd(P, P, P, P, P, P, P, P, P, 128, 128, 0.125, 1, 4, 4, 64,
                                        BF16, None, 1 << 30, None)
    assert rc == WS


def test_other_ops_validation(L):
    assert L.teeny_rope_fwd(P, P, 8, 9.21, 2, 12, BF16, None) == UNSUP  # 12 % 8
    assert L.teeny_rope_fwd(None, P, 8, 9.21, 2, 16, F32, None) == NULLP
    assert L.teeny_rope_fwd(P, P, 8, 9.21, 2, 24, F32, None) == UNSUP  # not a power of two
    assert L.teeny_transpose_heads(P, P, 0, 4, 1, 64, BF16, None) == SHAPE
    assert L.teeny_transpose_heads(P, P, 8, 4, 1, 64, BF16, None) == VALUE  # src == dst
    assert L.teeny_rmsnorm_fwd(P, P, None, P, 4, 64 * 8 * 32, 1e-5, BF16, None) == UNSUP
    assert L.teeny_fused_add_rmsnorm_fwd(P, P, P, P, None, P, 4, 16, 1e-6, F32, None) == NULLP
    assert L.teeny_fused_add_rmsnorm_bwd(P, P, P, P, P, P, P, 4, 16, F32, None, 0, None) == WS
    assert L.teeny_swiglu_fwd(P, P, 0, 8, F32, None) == SHAPE
    assert L.teeny_token_embed_fwd(P, P, P, 4, 16, 10, BF16, F32, None) == UNSUP  # ids dtype


def test_add_validation(L):
    assert L.teeny_add(None, P, P, 16, BF16, None) == NULLP
    assert L.teeny_add(P, P, P, 0, BF16, None) == SHAPE
    assert L.teeny_add(P + 2, P, P, 16, BF16, None) == VALUE  # not 16-byte aligned
    assert L.teeny_add(P, P, P, 16, 9, None) == UNSUP


def test_decode_ops_validation(L):
    # linear: any M; the matrix-core GEMM needs N % 64 and K % 64 (the
    # decode-step kernels, M <= 16, N % 128 and K % 128)
    assert L.teeny_linear_bf16(P, P, P, 17, 96, 128, None) == UNSUP
    assert L.teeny_linear_bf16(P, P, P, 16, 64, 96, None) == UNSUP
    assert L.teeny_linear_bf16(P, P, P, 300, 128, 4100, None) == UNSUP
    assert L.teeny_linear_bf16(P, P, P, 300, 128, 1 << 22, None) == SHAPE  # 32-bit offsets
    # linear_swiglu: the GEMM needs F % 32 and K % 64 (the decode kernel,
    # M <= 16, F % 64 and K % 128)
    assert L.teeny_linear_swiglu_bf16(P, P, P, 17, 48, 128, None) == UNSUP
    assert L.teeny_linear_swiglu_bf16(P, P, P, 300, 64, 96, None) == UNSUP
    assert L.teeny_linear_swiglu_bf16(P, P, P, 300, 64, 1 << 22, None) == SHAPE
    assert L.teeny_linear_swiglu_bf16(P, None, P, 300, 64, 128, None) == NULLP
    assert L.teeny_linear_bf16(None, P, P, 16, 128, 128, None) == NULLP
    assert L.teeny_linear_bf16(P, P, P, 0, 128, 128, None) == SHAPE
    assert L.teeny_linear_swiglu_bf16(P, P, P, 4, 48, 128, None) == UNSUP
    assert L.teeny_linear_partials_bf16(P, P, P, 4, 128, 4096, 1000, None) == VALUE
    assert L.teeny_linear_partials_bf16(P, P, P, 4, 128, 4096, 0, None) == VALUE
    assert L.teeny_linear_partials_count(4096, 1024) == 4
    assert L.teeny_linear_partials_count(14336, 2048) == 7
    assert L.teeny_linear_partials_count(4096, 8192) == 1
    assert L.teeny_fused_add_rmsnorm_partials_fwd(P, 0, P, P, P, P, P, 4, 1024, 1e-5, BF16,
                                                  None) == SHAPE
    assert L.teeny_fused_add_rmsnorm_partials_fwd(None, 2, P, P, P, P, P, 4, 1024, 1e-5, BF16,
                                                  None) == NULLP
    assert L.teeny_qkv_rope_split_partials_dev(P, 2, P, P, P, 4, 1, None, 64, 8, 2, 64,
                                               9.21, BF16, None) == NULLP
    assert L.teeny_qkv_rope_split_partials_dev(P, 2, P, P, P, 4, 1, P, 64, 8, 3, 64,
                                               9.21, BF16, None) == SHAPE  # 8 % 3
    assert L.teeny_argmax_rows(None, P, 4, 10, BF16, None) == NULLP
    assert L.teeny_argmax_rows(P, P, 0, 10, BF16, None) == SHAPE


def test_decode_qkv_attention_validation(L):
    def call(**kw):
        a = dict(parts=P, n=4, k=P, v=P, o=P, b=2, hq=32, hkv=8, d=128, cl=640, pos=P,
                 lnb=13.1, scale=0.088, dtype=BF16)
        a.update(kw)
        return L.teeny_decode_qkv_attention_dev(a["parts"], a["n"], a["k"], a["v"], a["o"], a["b"],
                                                a["hq"], a["hkv"], a["d"], a["cl"], a["pos"],
                                                a["lnb"], a["scale"], a["dtype"], None)
    assert call(parts=None) == NULLP
    assert call(pos=None) == NULLP
    assert call(dtype=F32) == UNSUP
    assert call(d=96) == UNSUP
    assert call(hq=64, hkv=1) == UNSUP  # 64 q heads per kv head: more than one product's rows
    assert call(hq=6, hkv=4) == SHAPE
    assert call(n=0) == SHAPE
    assert call(scale=-1.0) == VALUE
    assert call(lnb=float("nan")) == VALUE


def test_fa2_32bit_row_offsets(L):
    """bf16 kernels address a head's rows through 32-bit buffer offsets: a
    head of n_ctx * D * 2 >= 2^31 bytes (Q or dO of 8.4M rows at D = 128,
    fewer than 2^31 elements in all) is refused before any launch, on the
    query side as on the key side."""
    big = 8_400_000  # 8.4M * 128 * 2 B = 2.15e9 B; 8.4M * 128 = 1.08e9 elements
    assert fwd(L, nq=big, nk=128, hq=1, hkv=1, d=128) == SHAPE
    assert fwd(L, nq=128, nk=big, hq=1, hkv=1, d=128) == SHAPE
    ws = 1 << 30
    for nq, nk in ((big, 128), (128, big)):
        rc = L.teeny_causal_flash_attn2_bwd(P, P, P, P, P, P, P, P, P, nq, nk, 0.088, 1, 1, 1,
                                            128, BF16, P, ws, None)
        assert rc == SHAPE, (nq, nk)
    # fp32 kernels index elements, not byte ranges: the element bound applies
    assert fwd(L, nq=big, nk=128, hq=1, hkv=1, d=128, dtype=F32) != SHAPE


def test_decode_qkv_attention_32bit_cache_offsets(L):
    """One (b, kv head) cache slab of cache_len * D * 2 >= 2^31 bytes is refused."""
    rc = L.teeny_decode_qkv_attention_dev(P, 1, P, P, P, 1, 1, 1, 128, 8_400_000, P, 13.1,
                                          0.088, BF16, None)
    assert rc == SHAPE
    rc = L.teeny_decode_qkv_attention_dev(P, 1, P, P, P, 1, 1, 1, 128, 4_000_000, P, 13.1,
                                          0.088, BF16, None)
    assert rc != SHAPE  # within range: fails later (no GPU here), not on the shape


def test_noalloc_needs_init(L):
    """The no-allocation backward loads and looks up nothing itself: without
    a device (here) it reports the HIP error, never a launch; its
    not-initialised code has its own text."""
    rc = L.teeny_causal_flash_attn2_bwd_noalloc(P, P, P, P, P, P, P, P, P, 128, 128, 0.125, 1,
                                                4, 4, 64, BF16, None)
    assert rc in (-5, NOT_INIT)
    assert "teeny_init" in L.teeny_strerror(NOT_INIT).decode()


def test_linear_f32_validation(L):
    """fp32 Linear (teeny_linear_f32 / teeny_gemm_f32): any M and N, K a
    multiple of 4, 16-byte aligned operands."""
    for fn in (L.teeny_linear_f32, L.teeny_gemm_f32):
        assert fn(None, P, P, 4, 8, 8, None) == NULLP
        assert fn(P, P, P, 0, 8, 8, None) == SHAPE
        assert fn(P, P, P, 4, 8, 6, None) == UNSUP
        assert fn(P + 4, P, P, 4, 8, 8, None) == VALUE
        assert fn(P, P + 8, P, 4, 8, 8, None) == VALUE


def test_stream_layout_validation(L):
    """The streaming layout (N % 16, K % 128, no overlap) and the linears
    that read it (the decode kernels' shapes only: M <= 16, N % 128 or
    F % 64, K % 128)."""
    Q = P + (1 << 30)  # a second buffer far from P
    assert L.teeny_linear_stream_layout_bf16(None, Q, 16, 128, None) == NULLP
    assert L.teeny_linear_stream_layout_bf16(P, Q, 0, 128, None) == SHAPE
    assert L.teeny_linear_stream_layout_bf16(P, Q, 24, 128, None) == UNSUP
    assert L.teeny_linear_stream_layout_bf16(P, Q, 16, 96, None) == UNSUP
    assert L.teeny_linear_stream_layout_bf16(P, P, 16, 128, None) == VALUE  # in place
    assert L.teeny_linear_stream_layout_bf16(P, P + 2 * 16 * 128 - 2, 16, 128, None) == VALUE
    assert L.teeny_linear_stream_layout_bf16(P, Q, 1 << 16, 1 << 16, None) == SHAPE
    assert L.teeny_linear_sl_bf16(None, P, P, 4, 128, 128, None) == NULLP
    assert L.teeny_linear_sl_bf16(P, P, P, 17, 128, 128, None) == UNSUP  # prompt sizes: row-major
    assert L.teeny_linear_sl_bf16(P, P, P, 4, 96, 128, None) == UNSUP
    assert L.teeny_linear_sl_bf16(P, P, P, 4, 128, 192, None) == UNSUP
    assert L.teeny_linear_swiglu_sl_bf16(P, P, P, 4, 96, 128, None) == UNSUP
    assert L.teeny_linear_swiglu_sl_bf16(P, P, P, 0, 64, 128, None) == SHAPE
    assert L.teeny_linear_partials_sl_bf16(P, P, P, 4, 128, 4096, 1000, None) == VALUE
    assert L.teeny_linear_partials_sl_bf16(P, P, P, 4, 128, 4096, 0, None) == VALUE
    assert L.teeny_linear_partials_sl_bf16(P, None, P, 4, 128, 4096, 512, None) == NULLP


def test_header_is_c(tmp_path):
    """include/teeny_hip.h is a C header: a C99 program that includes it
    compiles without warnings, links against libteeny_hip.so and calls it
    (what a cgo / bindgen / ctypes consumer relies on)."""
    import os
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no C compiler")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    libdir = os.path.join(root, "teenyformers_amd")
    src = tmp_path / "use_header.c"
    src.write_text('#include "teeny_hip.h"\n'
                   "int main(void) { return teeny_abi_version() == 1 ? 0 : 1; }\n")
    exe = tmp_path / "use_header"
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    subprocess.run([gcc, "-std=c99", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
                    "-I" + os.path.join(root, "include"), "-I" + os.path.join(rocm, "include"),
                    str(src), "-L" + libdir, "-lteeny_hip", "-Wl,-rpath," + libdir,
                    "-o", str(exe)], check=True)
    assert subprocess.run([str(exe)]).returncode == 0

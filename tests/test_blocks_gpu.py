"""The reference's own block fixtures through the HIP kernels, fp32.

tests/golden/encoder_block and decoder_block are the reference's
tests/fixtures (written by its tests/fixtures/generate.py:133-279 with RoPE
disabled): a pre-norm encoder block, whose self-attention is bidirectional,
and a decoder block with causal self-attention and cross-attention from 5
target rows to 7 encoder rows (Sq != Sk).  Here each block is composed from
the library's ops on the device (RMSNorm, the fp32 Linear, head transposes,
the fp32 flash-attention forward, residual adds, SwiGLU), in the reference
layers' order (src/layers/attention.rs:83-148 without RoPE,
src/layers/ffn.rs:47-56), and compared with the fixture's output at the
reference's kernel-test tolerance, 1e-4 (tests/kernel_execution.rs:36)."""
import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from teenyformers_amd import ops

pytestmark = pytest.mark.gpu

TOL = 1e-4
EPS = 1e-6  # the fixtures' RMSNorm eps (generate.py:136)


def _load(name):
    meta = json.load(open(os.path.join(O.GOLDEN, name, "meta.json")))
    w = {k: torch.from_numpy(O.load_fixture(f"{name}/{k.replace('.', '_')}.bin").reshape(s)).cuda()
         for k, s in meta["weights"].items()}
    return meta, w


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _attention(xq, xkv, wq, wk, wv, wo, H, causal):
    """Projections -> head transposes -> FA2 -> merge -> output projection,
    every step a library kernel (fp32)."""
    Dh = xq.shape[-1] // H
    q = ops.transpose_heads(ops.linear(xq, wq), H)
    k = ops.transpose_heads(ops.linear(xkv, wk), H)
    v = ops.transpose_heads(ops.linear(xkv, wv), H)
    o, _ = ops.flash_attn2_fwd(q, k, v, 1.0 / math.sqrt(Dh), causal=causal)
    return ops.linear(ops.merge_heads(o), wo)


def _ffn(x, norm_w, w_gate_up, w_down):
    n, _ = ops.rmsnorm(x, norm_w, EPS)
    return ops.linear(ops.swiglu(ops.linear(n, w_gate_up)), w_down)


def test_encoder_block_fixture(cuda):
    meta, w = _load("encoder_block")
    x = _dev(O.load_fixture("encoder_block/input.bin").reshape(meta["seq"], meta["d_model"]))
    H = meta["n_heads"]
    n1, _ = ops.rmsnorm(x, w["norm1.weight"], EPS)
    x2 = ops.add(x, _attention(n1, n1, w["wq.weight"], w["wk.weight"], w["wv.weight"],
                               w["wo.weight"], H, causal=False).contiguous())
    out = ops.add(x2, _ffn(x2, w["norm2.weight"], w["wgate_up.weight"], w["wdown.weight"])
                  .contiguous())
    want = O.load_fixture("encoder_block/output.bin").reshape(tuple(out.shape))
    err = float(np.abs(out.cpu().numpy() - want).max())
    print(f"encoder block fixture: max abs {err:.2e}", flush=True)
    assert err < TOL


def test_decoder_block_fixture(cuda):
    meta, w = _load("decoder_block")
    st, se, Dm, H = meta["seq_tgt"], meta["seq_enc"], meta["d_model"], meta["n_heads"]
    tgt = _dev(O.load_fixture("decoder_block/input_tgt.bin").reshape(st, Dm))
    enc = _dev(O.load_fixture("decoder_block/input_enc.bin").reshape(se, Dm))
    n1, _ = ops.rmsnorm(tgt, w["norm1.weight"], EPS)
    t = ops.add(tgt, _attention(n1, n1, w["wqs.weight"], w["wks.weight"], w["wvs.weight"],
                                w["wos.weight"], H, causal=True).contiguous())
    n2, _ = ops.rmsnorm(t, w["norm2.weight"], EPS)
    # cross-attention: 5 target rows attend to 7 encoder rows, no mask
    t = ops.add(t, _attention(n2, enc, w["wqc.weight"], w["wkc.weight"], w["wvc.weight"],
                              w["woc.weight"], H, causal=False).contiguous())
    out = ops.add(t, _ffn(t, w["norm3.weight"], w["wgate_up.weight"], w["wdown.weight"])
                  .contiguous())
    want = O.load_fixture("decoder_block/output.bin").reshape(tuple(out.shape))
    err = float(np.abs(out.cpu().numpy() - want).max())
    print(f"decoder block fixture: max abs {err:.2e}", flush=True)
    assert err < TOL

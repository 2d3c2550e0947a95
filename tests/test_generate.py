"""Checkpoint loading and the generation CLI (examples/llama_generate.rs,
src/loader.rs).  The CPU tests write tiny HF-format checkpoints with the
safetensors library and read them back; the GPU test runs the CLI end to end
on such a checkpoint with a word-level tokenizer built here."""
import io
import json
import os
from contextlib import redirect_stdout

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from teenyformers_amd import generate, llama

TINY = dict(d_model=256, n_heads=4, n_layers=2, vocab_size=96, eps=1e-5, rope_base=1e4,
            intermediate_size=256, n_kv_heads_=2)


def _hf_tensors(cfg, seed=0):
    """HF-named tensors: separate q/k/v and gate/up, plus an (unused) lm_head."""
    g = torch.Generator().manual_seed(seed)
    d, D, Hq, Hkv, F_ = cfg.d_model, cfg.head_dim(), cfg.n_heads, cfg.n_kv_heads(), cfg.d_ff()

    def r(*s):
        return (0.02 * torch.randn(s, generator=g)).to(torch.bfloat16)

    t = {"model.embed_tokens.weight": r(cfg.vocab_size, d), "model.norm.weight": 1 + r(d),
         "lm_head.weight": r(cfg.vocab_size, d)}
    for i in range(cfg.n_layers):
        p = f"model.layers.{i}."
        t[p + "input_layernorm.weight"] = 1 + r(d)
        t[p + "post_attention_layernorm.weight"] = 1 + r(d)
        t[p + "self_attn.q_proj.weight"] = r(Hq * D, d)
        t[p + "self_attn.k_proj.weight"] = r(Hkv * D, d)
        t[p + "self_attn.v_proj.weight"] = r(Hkv * D, d)
        t[p + "self_attn.o_proj.weight"] = r(d, Hq * D)
        t[p + "mlp.gate_proj.weight"] = r(cfg.d_ff(), d)
        t[p + "mlp.up_proj.weight"] = r(cfg.d_ff(), d)
        t[p + "mlp.down_proj.weight"] = r(d, cfg.d_ff())
    return t


def _write_checkpoint(path, cfg, tensors):
    os.makedirs(path, exist_ok=True)
    names = sorted(tensors)
    half = len(names) // 2  # two shards, as large checkpoints are split
    save_file({k: tensors[k].contiguous() for k in names[:half]},
              os.path.join(path, "model-00001-of-00002.safetensors"))
    save_file({k: tensors[k].contiguous() for k in names[half:]},
              os.path.join(path, "model-00002-of-00002.safetensors"))
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump({"hidden_size": cfg.d_model, "num_attention_heads": cfg.n_heads,
                   "num_hidden_layers": cfg.n_layers, "vocab_size": cfg.vocab_size,
                   "rms_norm_eps": cfg.eps, "rope_theta": cfg.rope_base,
                   "intermediate_size": cfg.intermediate_size,
                   "num_key_value_heads": cfg.n_kv_heads_}, f)


def test_load_hf_weights_fuses_projections(tmp_path):
    cfg = llama.LlamaConfig(**TINY)
    t = _hf_tensors(cfg)
    _write_checkpoint(str(tmp_path), cfg, t)
    cfg2 = llama.LlamaConfig.from_hf_json(str(tmp_path / "config.json"))
    assert cfg2.n_kv_heads() == 2 and cfg2.d_ff() == 256 and cfg2.head_dim() == 64
    w = llama.load_hf_weights(cfg2, str(tmp_path), dtype=torch.float32, device="cpu")
    p = "model.layers.1."
    # gate first, then up (src/loader.rs:49-55); q | k | v for the fused projection
    assert torch.equal(w[p + "mlp.gate_up_proj.weight"],
                       torch.cat([t[p + "mlp.gate_proj.weight"],
                                  t[p + "mlp.up_proj.weight"]]).float())
    assert torch.equal(w[p + "self_attn.qkv_proj.weight"],
                       torch.cat([t[p + "self_attn.q_proj.weight"],
                                  t[p + "self_attn.k_proj.weight"],
                                  t[p + "self_attn.v_proj.weight"]]).float())
    assert torch.equal(w["model.norm.weight"], t["model.norm.weight"].float())
    assert "lm_head.weight" not in w  # tied embedding (src/llama.rs:80)
    # bf16 -> bf16 is exact
    wb = llama.load_hf_weights(cfg2, str(tmp_path), dtype=torch.bfloat16, device="cpu")
    assert torch.equal(wb["model.embed_tokens.weight"], t["model.embed_tokens.weight"])


def test_load_hf_weights_errors(tmp_path):
    cfg = llama.LlamaConfig(**TINY)
    with pytest.raises(FileNotFoundError):
        llama.load_hf_weights(cfg, str(tmp_path), device="cpu")
    t = _hf_tensors(cfg)
    del t["model.layers.0.mlp.up_proj.weight"]
    _write_checkpoint(str(tmp_path), cfg, t)
    with pytest.raises(KeyError, match="up_proj"):
        llama.load_hf_weights(cfg, str(tmp_path), device="cpu")
    bad = llama.LlamaConfig(**{**TINY, "intermediate_size": 512})
    t = _hf_tensors(cfg)
    _write_checkpoint(str(tmp_path), cfg, t)
    with pytest.raises(ValueError, match="shape"):
        llama.load_hf_weights(bad, str(tmp_path), device="cpu")


def test_xorshift_known_answers():
    """Marsaglia's xorshift64 (13, 7, 17) from state 1: 1082269761, then
    1152992998833853505 (the published first outputs of this triple)."""
    rng = generate.XorShift(1)
    rng.next_unit()
    assert rng.s == 1082269761
    rng.next_unit()
    assert rng.s == 1152992998833853505


def test_temperature_sample():
    rng = generate.XorShift(7)
    # one overwhelming logit: always chosen
    lg = np.zeros(50, np.float32)
    lg[31] = 100.0
    assert all(generate.temperature_sample(lg, 1.0, rng) == 31 for _ in range(20))
    # two logits with probabilities 1/4 and 3/4: index 0 exactly when r < 1/4
    lg2 = np.array([0.0, np.log(3.0)], np.float32)
    for _ in range(50):
        probe = generate.XorShift(rng.s)
        r = probe.next_unit()
        want = 0 if r < np.float32(0.25) else 1
        if abs(float(r) - 0.25) > 1e-6:
            assert generate.temperature_sample(lg2, 1.0, rng) == want
        else:
            rng.next_unit()


class _Vocab:
    def __init__(self, v):
        self.v = v

    def get_vocab(self, with_added_tokens=True):
        return self.v


def test_eos_id():
    assert generate.eos_id(_Vocab({"a": 0, "<|eot_id|>": 9, "</s>": 4})) == 4
    assert generate.eos_id(_Vocab({"a": 0, "<|eot_id|>": 9})) == 9
    assert generate.eos_id(_Vocab({"a": 0})) == 2


@pytest.mark.gpu
def test_generate_cli_greedy_matches_model(tmp_path, cuda):
    """The CLI on a checkpoint prints the prompt and the greedy continuation
    the model's own KV-cached generate() produces."""
    from tokenizers import Tokenizer, models, pre_tokenizers

    cfg = llama.LlamaConfig(**TINY)
    _write_checkpoint(str(tmp_path), cfg, _hf_tensors(cfg, seed=3))
    words = [f"w{i}" for i in range(cfg.vocab_size)]
    tok = Tokenizer(models.WordLevel({w: i for i, w in enumerate(words)}, unk_token="w0"))
    tok.pre_tokenizer = pre_tokenizers.Whitespace()
    tok.save(str(tmp_path / "tokenizer.json"))
    prompt = "w5 w17 w3 w60"
    buf = io.StringIO()
    with redirect_stdout(buf):
        assert generate.main(["--model-dir", str(tmp_path), "--prompt", prompt,
                              "--max-new-tokens", "6"]) == 0
    w = llama.load_hf_weights(cfg, str(tmp_path))
    ids = torch.tensor([[5, 17, 3, 60]], device="cuda")
    want = llama.Llama(cfg, w).generate(ids, 6)[0].tolist()
    # no end-of-sequence token in this vocabulary except id 2 (the fallback)
    if 2 in want:
        want = want[:want.index(2)]
    assert buf.getvalue() == prompt + "".join(words[i] for i in want) + "\n"


def test_config_d_ff_default_rounding():
    """Without intermediate_size, d_ff = ceil(ceil(8 d / 3) / 64) * 64
    (src/config.rs:146-153), the rule the reference's own config test pins
    (tests/graph_construction.rs:55-61: d 128 -> 384, d 512 -> a multiple of
    64), checked against exact rational arithmetic for every d to 8192."""
    from fractions import Fraction
    import math as _m

    assert llama.LlamaConfig(d_model=128).d_ff() == 384
    assert llama.LlamaConfig(d_model=512).d_ff() == 1408
    assert llama.LlamaConfig().d_ff() == 10944  # the default d 4096
    assert llama.LlamaConfig(d_model=4096, intermediate_size=14336).d_ff() == 14336
    for d in range(1, 8193):
        want = _m.ceil(Fraction(_m.ceil(Fraction(8 * d, 3)), 64)) * 64
        assert llama.LlamaConfig(d_model=d).d_ff() == want, d

"""Autoregressive generation with the Llama model on one MI355X.

The counterpart of the reference's examples/llama_generate.rs: a HF model
directory (config.json, tokenizer.json, *.safetensors) and a prompt, greedy
or temperature sampling, stop at the end-of-sequence token.  Unlike the
reference, which recomputes the whole sequence every step
(llama_generate.rs:373-391), the prompt fills a KV cache once and each new
token is one decode step; greedy steps are captured in a HIP graph.  GQA
checkpoints are accepted (the reference refuses them, :131-142).

  python -m teenyformers_amd.generate --model-dir DIR --prompt "The quick brown fox"

Without a checkpoint, --preset llama3-8b runs the Llama-3-8B shape with
random N(0, 0.02) weights and random prompt ids, prints one JSON line of
timings, and is the workload of the decode kernel profiles:

  python -m teenyformers_amd.generate --preset llama3-8b --batch 16 --prompt-len 512
"""
from __future__ import annotations

import argparse
import json
import sys
import time

import numpy as np
import torch

from . import llama, ops

PRESETS = {
    "llama3-8b": dict(d_model=4096, n_heads=32, n_layers=32, vocab_size=128256, eps=1e-5,
                      rope_base=5e5, intermediate_size=14336, n_kv_heads_=8),
}


class XorShift:
    """The reference's sampler state and step (llama_generate.rs:262-266)."""

    MASK = (1 << 64) - 1

    def __init__(self, seed: int):
        self.s = seed & self.MASK

    def next_unit(self) -> np.float32:
        s = self.s
        s ^= (s << 13) & self.MASK
        s ^= s >> 7
        s ^= (s << 17) & self.MASK
        self.s = s
        return np.float32(s) / np.float32(self.MASK)


def temperature_sample(logits: np.ndarray, temp: float, rng: XorShift) -> int:
    """llama_generate.rs:254-275: softmax of logits / temp in f32, one
    uniform draw, the first index whose running sum exceeds it."""
    scaled = logits.astype(np.float32) / np.float32(temp)
    exps = np.exp(scaled - scaled.max()).astype(np.float32)
    probs = (exps / exps.sum(dtype=np.float32)).astype(np.float32)
    r = rng.next_unit()
    cum = np.float32(0.0)
    for i, p in enumerate(probs):
        cum = np.float32(cum + p)
        if r < cum:
            return i
    return len(probs) - 1


def eos_id(tok) -> int:
    """llama_generate.rs:349-356: the first of the usual EOS names, else 2."""
    vocab = tok.get_vocab(with_added_tokens=True)
    for name in ("</s>", "<|endoftext|>", "<eos>", "<|eot_id|>"):
        if name in vocab:
            return vocab[name]
    return 2


def generate_text(args) -> int:
    import os

    from tokenizers import Tokenizer

    cfg = llama.LlamaConfig.from_hf_json(os.path.join(args.model_dir, "config.json"))
    print(f"d_model={cfg.d_model} n_heads={cfg.n_heads} n_kv_heads={cfg.n_kv_heads()} "
          f"n_layers={cfg.n_layers} vocab={cfg.vocab_size} d_ff={cfg.d_ff()}", file=sys.stderr)
    dtype = torch.float32 if args.dtype == "f32" else torch.bfloat16
    w = llama.load_hf_weights(cfg, args.model_dir, dtype=dtype)
    model = llama.Llama(cfg, w)
    tok = Tokenizer.from_file(os.path.join(args.model_dir, "tokenizer.json"))
    ids = tok.encode(args.prompt, add_special_tokens=False).ids
    eos = eos_id(tok)
    print(args.prompt, end="", flush=True)
    prompt = torch.tensor([ids], dtype=torch.int64, device="cuda")
    cache, logits = model.prefill(prompt, len(ids) + args.max_new_tokens)
    if not args.no_stream_layout:
        model.stream_layout()
    rng = XorShift(args.seed)
    dg = None
    for step in range(args.max_new_tokens):
        if args.temperature == 0.0:
            if dg is None:
                nxt = int(ops.argmax_rows(logits).item())
            else:
                nxt = int(dg.ids.item())
        else:
            nxt = temperature_sample(logits[0].float().cpu().numpy(), args.temperature, rng)
        if nxt == eos:
            break
        print(tok.decode([nxt], skip_special_tokens=True), end="", flush=True)
        if step + 1 == args.max_new_tokens:
            break
        if args.temperature == 0.0:
            if dg is None:  # capture the greedy step once, then replay it
                dg = llama.DecodeGraph(model, cache, torch.tensor([[nxt]], device="cuda"))
            else:
                dg.replay()
        else:
            logits = model.decode_step(cache, torch.tensor([[nxt]], device="cuda"))
    print()
    return 0


def bench_preset(args) -> int:
    cfg = llama.LlamaConfig(**PRESETS[args.preset])
    w = llama.init_weights(cfg, dtype=torch.bfloat16, seed=args.seed)
    model = llama.Llama(cfg, w)
    g = torch.Generator(device="cuda").manual_seed(args.seed)
    ids = torch.randint(0, cfg.vocab_size, (args.batch, args.prompt_len), generator=g,
                        device="cuda")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    cache, logits = model.prefill(ids, args.prompt_len + args.max_new_tokens)
    torch.cuda.synchronize()
    prefill_ms = (time.perf_counter() - t0) * 1e3
    print(f"prefill {prefill_ms:.1f} ms", file=sys.stderr, flush=True)
    if not args.no_stream_layout:
        model.stream_layout()
    dg = llama.DecodeGraph(model, cache, ops.argmax_rows(logits).view(-1, 1))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.max_new_tokens - 1):
        dg.replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / max(1, args.max_new_tokens - 1)
    print(json.dumps({"preset": args.preset, "batch": args.batch, "prompt_len": args.prompt_len,
                      "new_tokens": args.max_new_tokens, "prefill_ms": round(prefill_ms, 2),
                      "decode_ms_per_step": round(ms, 3),
                      "decode_tokens_per_s": round(args.batch / ms * 1e3, 1)}), flush=True)
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--model-dir", help="config.json, tokenizer.json and *.safetensors")
    ap.add_argument("--prompt", default="The quick brown fox")
    ap.add_argument("--max-new-tokens", type=int, default=128)
    ap.add_argument("--temperature", type=float, default=0.0)
    ap.add_argument("--seed", type=int, default=42)
    ap.add_argument("--dtype", choices=["bf16", "f32"], default="bf16")
    ap.add_argument("--preset", choices=sorted(PRESETS), help="random weights, timing only")
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--prompt-len", type=int, default=512)
    ap.add_argument("--no-stream-layout", action="store_true",
                    help="decode from the row-major weights (saves one copy of them)")
    args = ap.parse_args(argv)
    if args.max_new_tokens < 1:
        ap.error("--max-new-tokens must be at least 1")
    if args.preset:
        return bench_preset(args)
    if not args.model_dir:
        ap.error("give --model-dir (a HF checkpoint) or --preset")
    return generate_text(args)


if __name__ == "__main__":
    sys.exit(main())

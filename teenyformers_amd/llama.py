"""Llama decoder model over the HIP ops: the reference's layers with batch,
GQA, a KV cache and bf16 weights.

Mirrors (reference file:line):
  LlamaConfig                     src/config.rs:62-179 (n_kv_heads honoured, unlike
                                  Llama::new at src/llama.rs:53)
  MultiHeadAttention.forward      src/layers/attention.rs:83-148: projections ->
                                  transpose_heads -> RoPE -> causal FA2 -> merge_heads -> o_proj
  FeedForward.forward             src/layers/ffn.rs:47-56: fused gate||up -> SwiGLU -> down
  LlamaBlock.forward              src/layers/llama_block.rs:55-65: x + attn(rms(x)), then
                                  + ffn(rms(.))
  Llama.forward                   src/llama.rs:65-81: embed -> blocks -> norm -> tied lm_head
  generate_recompute              examples/llama_generate.rs:373-391: greedy decoding by
                                  recomputing the whole sequence each step

MI355X-specific structure (same arithmetic):
  * q/k/v projections are one GEMM against the concatenated weight, and
    teeny_qkv_rope_split does the three head transposes, both RoPEs and the
    KV-cache write in one pass;
  * every residual add is fused into the next RMSNorm (teeny_fused_add_rmsnorm);
  * prefill runs the causal FA2 kernel over the cache; each decode step runs
    teeny_decode_attention over the cached keys;
  * Linear layers (teeny-core's external `Linear`, src/layers/mod.rs:54-58,
    y = x W^T with W [out, in]) run through the library's linear entry
    points: a prompt's products through hipBLASLt (teeny_linear_bf16 /
    teeny_linear_f32), and with at most 16 rows (a decode step) the
    weight-streaming kernels: gate_up fused with SwiGLU, and q|k|v, o and
    down split over K into fp32 slabs that the QKV split and the
    residual-add norms sum.  Decode steps of more than 16 sequences run the
    library's own GEMM (ops.own_gemm), the kernel a captured graph runs, so
    eager and graph-replayed steps compute the same bits.
"""
from __future__ import annotations

import dataclasses
import json
import math

import torch

from . import ops


@dataclasses.dataclass
class LlamaConfig:
    """src/config.rs:62-82; defaults from src/config.rs:165-179."""
    d_model: int = 4096
    n_heads: int = 32
    n_layers: int = 32
    vocab_size: int = 32000
    max_seq_len: int = 4096
    eps: float = 1e-5
    rope_base: float = 10000.0
    intermediate_size: int | None = None
    n_kv_heads_: int | None = None

    def head_dim(self) -> int:  # config.rs:138-140
        return self.d_model // self.n_heads

    def d_ff(self) -> int:  # config.rs:146-153: intermediate_size or ceil(8d/3 / 64) * 64
        if self.intermediate_size is not None:
            return self.intermediate_size
        raw = -(-8 * self.d_model // 3)
        return -(-raw // 64) * 64

    def softmax_scale(self) -> float:  # config.rs:156-158 (f32)
        return float(torch.tensor(1.0, dtype=torch.float32)
                     / torch.tensor(float(self.head_dim()), dtype=torch.float32).sqrt())

    def n_kv_heads(self) -> int:  # config.rs:161-163
        return self.n_kv_heads_ if self.n_kv_heads_ is not None else self.n_heads

    @classmethod
    def from_hf_json(cls, path: str) -> "LlamaConfig":
        """HF config.json subset (config.rs:84-134)."""
        with open(path) as f:
            hf = json.load(f)
        return cls(d_model=hf["hidden_size"], n_heads=hf["num_attention_heads"],
                   n_layers=hf["num_hidden_layers"], vocab_size=hf["vocab_size"],
                   max_seq_len=hf.get("max_position_embeddings", 4096),
                   eps=hf.get("rms_norm_eps", 1e-5), rope_base=hf.get("rope_theta", 10000.0),
                   intermediate_size=hf.get("intermediate_size"),
                   n_kv_heads_=hf.get("num_key_value_heads"))


def init_weights(cfg: LlamaConfig, dtype=torch.bfloat16, device="cuda", std: float = 0.02,
                 seed: int = 0) -> dict:
    """Random weights ~ N(0, std) (norm weights 1), HF names
    (src/llama.rs:66-80, src/layers/*.rs name scopes); q|k|v and gate|up are
    stored concatenated along rows, gate first (src/loader.rs:49-55)."""
    gen = torch.Generator(device=device).manual_seed(seed)
    D, Hq, Hkv, F_ = cfg.head_dim(), cfg.n_heads, cfg.n_kv_heads(), cfg.d_ff()
    d = cfg.d_model

    def rnd(*shape):
        return (torch.randn(shape, generator=gen, device=device, dtype=torch.float32) * std).to(dtype)

    w = {"model.embed_tokens.weight": rnd(cfg.vocab_size, d),
         "model.norm.weight": torch.ones(d, dtype=dtype, device=device)}
    for i in range(cfg.n_layers):
        p = f"model.layers.{i}."
        w[p + "input_layernorm.weight"] = torch.ones(d, dtype=dtype, device=device)
        w[p + "post_attention_layernorm.weight"] = torch.ones(d, dtype=dtype, device=device)
        w[p + "self_attn.qkv_proj.weight"] = rnd((Hq + 2 * Hkv) * D, d)
        w[p + "self_attn.o_proj.weight"] = rnd(d, Hq * D)
        w[p + "mlp.gate_up_proj.weight"] = rnd(2 * F_, d)
        w[p + "mlp.down_proj.weight"] = rnd(d, F_)
    return w


def load_hf_weights(cfg: LlamaConfig, model_dir: str, dtype=torch.bfloat16,
                    device="cuda") -> dict:
    """A HuggingFace Llama checkpoint (every *.safetensors file of model_dir)
    as this model's weights (src/loader.rs:31-56): gate_proj | up_proj are
    concatenated along rows into gate_up_proj (gate first, as the reference
    loader does), q_proj | k_proj | v_proj likewise into qkv_proj (this
    model's fused projection), and lm_head is the tied embedding
    (src/llama.rs:80; an lm_head.weight in the files is not used).  Tensors
    are read with the safetensors loader, which executes nothing from the
    file, and converted to `dtype`."""
    import glob
    import os

    from safetensors import safe_open

    paths = sorted(glob.glob(os.path.join(model_dir, "*.safetensors")))
    if not paths:
        raise FileNotFoundError(f"no .safetensors files found in {model_dir}")
    raw = {}
    for path in paths:
        with safe_open(path, framework="pt", device="cpu") as f:
            for k in f.keys():
                raw[k] = f.get_tensor(k)

    def get(name, shape):
        if name not in raw:
            raise KeyError(f"missing weight: {name}")
        t = raw[name]
        if tuple(t.shape) != tuple(shape):
            raise ValueError(f"{name}: shape {tuple(t.shape)}, the config needs {tuple(shape)}")
        return t

    d, D, Hq, Hkv, F_ = cfg.d_model, cfg.head_dim(), cfg.n_heads, cfg.n_kv_heads(), cfg.d_ff()
    w = {"model.embed_tokens.weight": get("model.embed_tokens.weight", (cfg.vocab_size, d)),
         "model.norm.weight": get("model.norm.weight", (d,))}
    for i in range(cfg.n_layers):
        p = f"model.layers.{i}."
        a, m = p + "self_attn.", p + "mlp."
        w[p + "input_layernorm.weight"] = get(p + "input_layernorm.weight", (d,))
        w[p + "post_attention_layernorm.weight"] = get(p + "post_attention_layernorm.weight",
                                                       (d,))
        w[a + "qkv_proj.weight"] = torch.cat([get(a + "q_proj.weight", (Hq * D, d)),
                                              get(a + "k_proj.weight", (Hkv * D, d)),
                                              get(a + "v_proj.weight", (Hkv * D, d))], 0)
        w[a + "o_proj.weight"] = get(a + "o_proj.weight", (d, Hq * D))
        w[m + "gate_up_proj.weight"] = torch.cat([get(m + "gate_proj.weight", (F_, d)),
                                                  get(m + "up_proj.weight", (F_, d))], 0)
        w[m + "down_proj.weight"] = get(m + "down_proj.weight", (d, F_))
    return {k: v.to(dtype).to(device).contiguous() for k, v in w.items()}


class KVCache:
    """Per-layer K/V caches [B, Hkv, capacity, D], zero-initialised (rows past
    the written prefix are masked by causality and must hold finite values)."""

    def __init__(self, cfg: LlamaConfig, batch: int, capacity: int, dtype, device="cuda"):
        shape = (batch, cfg.n_kv_heads(), capacity, cfg.head_dim())
        self.k = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(cfg.n_layers)]
        self.v = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(cfg.n_layers)]
        self.capacity = capacity
        self.length = 0


class Llama:
    """Forward passes of the Llama model (src/llama.rs:40-82) on the HIP ops."""

    def __init__(self, cfg: LlamaConfig, weights: dict):
        self.cfg = cfg
        self.w = weights
        self.decode_ws = None
        self.sw = {}  # streaming-layout copies of the decode weights (stream_layout)
        self._cs = None  # RoPE (cos, sin) table of the bf16 prompt attention

    def stream_layout(self) -> "Llama":
        """Give the weights that one-token steps stream (each layer's qkv, o,
        gate_up and down projections and the tied lm_head) a streaming-layout
        copy (ops.StreamWeight): the decode linears then read 1 KiB per load
        instruction, with the same outputs; prompt-sized products keep the
        row-major weights.  Costs one more copy of those weights.  bf16 only;
        weights whose shape the layout does not take are left as they are.
        The copies are made once: after changing the weights in place, clear
        self.sw and call this again."""
        names = ["model.embed_tokens.weight"]
        for i in range(self.cfg.n_layers):
            p = f"model.layers.{i}."
            names += [p + "self_attn.qkv_proj.weight", p + "self_attn.o_proj.weight",
                      p + "mlp.gate_up_proj.weight", p + "mlp.down_proj.weight"]
        for n in names:
            w = self.w[n]
            if (n not in self.sw and w.dtype == torch.bfloat16 and w.is_cuda
                    and w.shape[0] % 16 == 0 and w.shape[1] % 128 == 0):
                self.sw[n] = ops.StreamWeight(w)
        return self

    def _lw(self, name: str):
        """The weight of a linear layer: its StreamWeight if stream_layout()
        made one, else the tensor."""
        return self.sw.get(name, self.w[name])

    # -- one block (src/layers/llama_block.rs:55-65) -------------------------
    def _attention(self, i: int, n1: torch.Tensor, cache: KVCache, pos0) -> torch.Tensor:
        """src/layers/attention.rs:83-148 with GQA and a KV cache.  pos0: an int,
        or (one-token decode in a captured graph) an int32 device tensor."""
        cfg, w = self.cfg, self.w
        B, S, d = n1.shape
        Hq, Hkv, D = cfg.n_heads, cfg.n_kv_heads(), cfg.head_dim()
        p = f"model.layers.{i}.self_attn."
        # [B, S, (Hq+2Hkv) D]; K-split fp32 slabs at decode sizes
        qkv = ops.linear_split(n1, self._lw(p + "qkv_proj.weight"))
        scale = cfg.softmax_scale()
        if isinstance(pos0, torch.Tensor) and self._fused_decode(qkv, cache):
            # one launch: QKV split, RoPE, cache write and attention
            o = ops.decode_qkv_attention(qkv, cache.k[i], cache.v[i], pos0, Hq, Hkv,
                                         cfg.rope_base, scale)
            return ops.linear_split(o.view(B, 1, Hq * D), self._lw(p + "o_proj.weight"))
        if (not isinstance(pos0, torch.Tensor) and pos0 == 0
                and not isinstance(qkv, ops.Partials) and qkv.dtype == torch.bfloat16):
            # bf16 prompt: K and V into the cache; the attention reads the q
            # heads from qkv, rotates them as it loads them and writes the
            # merged-heads layout (the same bits as the split into a Q
            # buffer, the forward and merge_heads, with Q and O written and
            # read once fewer)
            ops.qkv_rope_split(qkv, None, cache.k[i], cache.v[i], 0, Hq, Hkv, cfg.rope_base)
            att, _ = ops.flash_attn2_fwd_qkv(qkv, self._rope_table(S, n1.device), cache.k[i],
                                             cache.v[i], Hq, scale, causal=True)
            return ops.linear_split(att, self._lw(p + "o_proj.weight"))
        q = torch.empty((B, Hq, S, D), dtype=n1.dtype, device=n1.device)
        ops.qkv_rope_split(qkv, q, cache.k[i], cache.v[i], pos0, Hq, Hkv, cfg.rope_base)
        if isinstance(pos0, torch.Tensor):  # graph decode: the position is on the device
            if S != 1:
                raise ValueError("a device position is for one-token decode steps")
            o = ops.decode_attention(q.view(B, Hq, D), cache.k[i], cache.v[i], cache.capacity,
                                     scale, workspace=self._decode_ws(B, cache, n1.device),
                                     n_past=pos0).view(B, Hq, 1, D)
        elif S == 1 and pos0 > 0:  # decode: the new row sees every cached key
            o = ops.decode_attention(q.view(B, Hq, D), cache.k[i], cache.v[i], pos0 + 1, scale,
                                     workspace=self._decode_ws(B, cache, n1.device)
                                     ).view(B, Hq, 1, D)
        else:
            if pos0 != 0:
                raise ValueError("prefill must start at position 0")
            # causal FA2 over the cache: keys past S are masked (key > query);
            # bf16 writes the merged-heads layout itself (one launch, one pass
            # over O fewer than the forward and then merge_heads)
            if q.dtype == torch.bfloat16:
                att, _ = ops.flash_attn2_fwd_merged(q, cache.k[i], cache.v[i], scale, causal=True)
                return ops.linear_split(att, self._lw(p + "o_proj.weight"))
            o, _ = ops.flash_attn2_fwd(q, cache.k[i], cache.v[i], scale, causal=True)
        # one position: [B, Hq, 1, D] is already the merged [B, 1, Hq D] layout
        att = o.view(B, S, Hq * D) if S == 1 else ops.merge_heads(o)
        return ops.linear_split(att, self._lw(p + "o_proj.weight"))

    def _rope_table(self, n: int, device) -> torch.Tensor:
        """RoPE's (cos, sin) for positions 0 .. n-1 at least (kept, grown to
        a power of two)."""
        cs, D = self._cs, self.cfg.head_dim()
        if cs is None or cs.numel() < n * D or cs.device != device:
            m = max(32, 1 << max(0, n - 1).bit_length())
            cs = self._cs = ops.rope_table(m, D, self.cfg.rope_base, device)
        return cs

    def _fused_decode(self, qkv, cache: KVCache) -> bool:
        """Whether a one-token step runs teeny_decode_qkv_attention_dev: bf16
        K-split QKV slabs, D 64 or 128, up to 32 q heads per kv head, and a
        cache short enough for one workgroup per (b, kv head)."""
        cfg = self.cfg
        return (isinstance(qkv, ops.Partials) and qkv.dtype == torch.bfloat16
                and cfg.head_dim() in (64, 128) and cfg.n_heads // cfg.n_kv_heads() <= 32
                and cache.capacity <= 4096)

    def _decode_ws(self, B: int, cache: KVCache, device) -> torch.Tensor:
        """Split-K workspace for decode attention over the whole cache."""
        need = ops._lib.lib().teeny_decode_attention_workspace_bytes(
            B, self.cfg.n_heads, cache.capacity, self.cfg.head_dim())
        if self.decode_ws is None or self.decode_ws.numel() < need:
            self.decode_ws = torch.empty(need, dtype=torch.uint8, device=device)
        return self.decode_ws

    def _ffn(self, i: int, n2: torch.Tensor) -> torch.Tensor:
        """src/layers/ffn.rs:47-56."""
        p = f"model.layers.{i}.mlp."
        f = ops.linear_swiglu(n2, self._lw(p + "gate_up_proj.weight"))
        return ops.linear_split(f, self._lw(p + "down_proj.weight"))

    def hidden(self, ids: torch.Tensor, cache: KVCache, pos0, trace: list | None = None
               ) -> torch.Tensor:
        """Final-norm hidden states [B, S, d] for ids [B, S] at positions pos0..,
        appending the new keys/values to `cache` (pos0 may be an int32 device
        tensor for one-token steps; cache.length is then left to the caller).
        trace: if a list, each block appends (x, attn, x + attn, ffn): its
        input residual stream, the attention sub-layer's output, the stream
        after the attention add, and the FFN output (the block's output is
        the sum of the last two)."""
        cfg, w = self.cfg, self.w
        x = ops.token_embed(ids.to(torch.int32).contiguous(), w["model.embed_tokens.weight"])
        eps = cfg.eps
        pos = pos0
        if ids.shape[1] == 1 and not isinstance(pos0, torch.Tensor) and pos0 > 0:
            # a one-token step takes its position from device memory, as the
            # captured graph does, so both run the same kernels
            pos = torch.tensor([pos0], dtype=torch.int32, device=ids.device)
        delta = None
        for i in range(cfg.n_layers):
            p = f"model.layers.{i}."
            if delta is None:
                n1, _ = ops.rmsnorm(x, w[p + "input_layernorm.weight"], eps, want_rstd=False)
            else:  # x = x + ffn(...) fused into this block's input norm
                n1, x, _ = ops.fused_add_rmsnorm(delta, x, w[p + "input_layernorm.weight"], eps)
            x_in = x
            a = self._attention(i, n1, cache, pos)
            n2, x, _ = ops.fused_add_rmsnorm(a, x, w[p + "post_attention_layernorm.weight"], eps)
            delta = self._ffn(i, n2)
            if trace is not None:
                trace.append((x_in, a, x, delta))
        y, _, _ = ops.fused_add_rmsnorm(delta, x, w["model.norm.weight"], eps)
        if not isinstance(pos0, torch.Tensor):
            cache.length = pos0 + ids.shape[1]
        return y

    def logits(self, h: torch.Tensor) -> torch.Tensor:
        """Tied lm_head (src/layers/embedding.rs:159-167): h @ E^T."""
        return ops.linear(h, self._lw("model.embed_tokens.weight"))

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        """All-position logits [B, S, vocab] (src/llama.rs:65-81)."""
        B, S = ids.shape
        cache = KVCache(self.cfg, B, S, self.w["model.norm.weight"].dtype, ids.device)
        return self.logits(self.hidden(ids, cache, 0))

    # -- generation -----------------------------------------------------------
    def prefill(self, ids: torch.Tensor, capacity: int) -> tuple[KVCache, torch.Tensor]:
        """Prompt pass: returns the cache and the last position's logits."""
        B, S = ids.shape
        cache = KVCache(self.cfg, B, capacity, self.w["model.norm.weight"].dtype, ids.device)
        h = self.hidden(ids, cache, 0)
        return cache, self.logits(h[:, -1])

    def decode_step(self, cache: KVCache, ids: torch.Tensor) -> torch.Tensor:
        """One token per sequence (ids [B, 1]) -> next-token logits [B, vocab]."""
        with ops.own_gemm():  # the kernels of the graph-captured step
            h = self.hidden(ids, cache, cache.length)
            return self.logits(h[:, -1])

    def generate(self, prompt: torch.Tensor, n_new: int) -> torch.Tensor:
        """Greedy decoding with the KV cache -> generated ids [B, n_new]."""
        cache, logits = self.prefill(prompt, prompt.shape[1] + n_new)
        out = []
        for _ in range(n_new):
            nxt = ops.argmax_rows(logits).view(-1, 1)  # greedy (llama_generate.rs:252-257)
            out.append(nxt)
            if len(out) == n_new:
                break
            logits = self.decode_step(cache, nxt)
        return torch.cat(out, dim=1)

    def generate_graph(self, prompt: torch.Tensor, n_new: int) -> torch.Tensor:
        """generate(), with the decode step captured once in a HIP graph and
        replayed (same ids; no per-step launch overhead)."""
        cache, logits = self.prefill(prompt, prompt.shape[1] + n_new)
        first = ops.argmax_rows(logits).view(-1, 1)
        if n_new == 1:
            return first
        dg = DecodeGraph(self, cache, first)  # runs decode step 1 while capturing
        out = [first, dg.ids.clone()]
        while len(out) < n_new:
            dg.replay()
            out.append(dg.ids.clone())
        return torch.cat(out, dim=1)

    def generate_recompute(self, prompt: torch.Tensor, n_new: int) -> torch.Tensor:
        """The reference's method (examples/llama_generate.rs:373-391): every
        step recomputes the whole sequence and takes the last row's argmax."""
        seq = prompt
        out = []
        for _ in range(n_new):
            B, S = seq.shape
            cache = KVCache(self.cfg, B, S, self.w["model.norm.weight"].dtype, seq.device)
            h = self.hidden(seq, cache, 0)
            nxt = ops.argmax_rows(self.logits(h[:, -1])).view(-1, 1)
            out.append(nxt)
            seq = torch.cat([seq, nxt], dim=1)
        return torch.cat(out, dim=1)


def block_forward(cfg: LlamaConfig, w: dict, x: torch.Tensor, layer: int = 0) -> torch.Tensor:
    """One LlamaBlock forward, x [B, S, d] -> [B, S, d] (src/layers/llama_block.rs:55-65)."""
    model = Llama(cfg, w)
    B, S, d = x.shape
    cache = KVCache(dataclasses.replace(cfg, n_layers=layer + 1), B, S, x.dtype, x.device)
    p = f"model.layers.{layer}."
    n1, _ = ops.rmsnorm(x, w[p + "input_layernorm.weight"], cfg.eps, want_rstd=False)
    a = model._attention(layer, n1, cache, 0)
    n2, x2, _ = ops.fused_add_rmsnorm(a, x, w[p + "post_attention_layernorm.weight"], cfg.eps)
    f = model._ffn(layer, n2)
    return ops.add(x2, f)


def prefill_flops(cfg: LlamaConfig, batch: int, seq: int, last_logits_only: bool = True) -> float:
    """Matrix FLOPs of a prefill: 2 * params * tokens for the layers, causal
    attention 4 * S^2/2 * Hq * D per layer and sequence, and the lm_head."""
    d, D, Hq, Hkv, F_ = cfg.d_model, cfg.head_dim(), cfg.n_heads, cfg.n_kv_heads(), cfg.d_ff()
    per_layer = d * (Hq + 2 * Hkv) * D + Hq * D * d + d * 2 * F_ + F_ * d
    tokens = batch * seq
    f = 2.0 * per_layer * tokens * cfg.n_layers
    f += cfg.n_layers * batch * 4.0 * seq * seq / 2 * Hq * D
    f += 2.0 * d * cfg.vocab_size * (batch if last_logits_only else tokens)
    return f


class DecodeGraph:
    """One greedy decode step (embed, every block with the KV cache, final
    norm, tied lm_head on the last position, argmax) captured in a HIP graph.
    The step reads its ids from `ids` [B, 1] (int64) and the cache length
    from `pos` (int32, device); replay() writes the next ids into `ids`,
    appends one cache row and advances `pos`.  The constructor runs the first
    step eagerly on a side stream (the capture needs its libraries warmed up)
    and then captures it, so after construction `ids` holds step 1's output
    and `first_logits` its logits.  `logits` [B, vocab] holds the last
    replayed step's logits.  trace: a list that the captured step's blocks
    append their sub-layer tensors to (as Llama.hidden's trace); after each
    replay they hold that step's values.  Positions past the cache capacity
    are not written (the kernels check)."""

    def __init__(self, model: Llama, cache: KVCache, ids: torch.Tensor,
                 trace: list | None = None):
        self.model, self.cache = model, cache
        self.ids = ids.to(torch.int64).clone()
        self.pos = torch.full((1,), cache.length, dtype=torch.int32, device=ids.device)
        model._decode_ws(ids.shape[0], cache, ids.device)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self._step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.first_logits = self.logits
        cache.length += 1
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._step(trace)

    def _step(self, trace: list | None = None):
        m = self.model
        # the eager first step runs the kernels the capture records (above 16
        # sequences the library's own GEMM, as teeny_linear_bf16 under capture)
        with ops.own_gemm():
            h = m.hidden(self.ids, self.cache, self.pos, trace=trace)
            self.logits = m.logits(h[:, -1])
            # the greedy choice lands in the ids the next replay embeds (the
            # embedding read them at the start of this step)
            ops.argmax_rows(self.logits, out=self.ids.view(-1))
        self.pos.add_(1)

    def replay(self):
        if self.cache.length >= self.cache.capacity:
            raise RuntimeError("KV cache is full")
        self.graph.replay()
        self.cache.length += 1

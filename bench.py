"""Benchmark of the attention hot path on one MI355X.

A step is one causal flash-attention-2 forward + backward (bf16 in, fp32
accumulate) over B=8, H=32 (MHA), S=4096, D=128, the headline shape; inputs
are resident in HBM before timing.  Prints one JSON line:
  value       whole-step throughput in TFLOP/s (algorithmic: causal forward
              4*B*H*S^2*D/2, backward 2.5x that)
  roofline    the dominant kernel (most summed time) measured with HIP events
              recorded on its launch stream during the timed steps; traffic =
              that kernel's HBM bytes per launch from the committed rocprofv3
              FETCH_SIZE / WRITE_SIZE summary (profiles/*_hbm_traffic.md)
  cpu_baseline the oracle's restatement of the reference kernels (fp32,
              every key of every row, as the reference loops) timed on a
              sample of heads on this host's cores
  detail      per-op numbers (forward, backward, each kernel), plus the other
              configurations: long-context GQA FA2 (B1 Hq64 Hkv8 D128,
              S=16384 and the ragged 8191, 1% of K rows x8), the library's
              GEMM at the Llama prompt shapes beside hipBLASLt, one Llama block
              forward (B4 S2048 d2048, Hq32/Hkv8, F8192, bf16), and the
              Llama-3-8B-shaped model (32 layers, d4096, Hq32/Hkv8, F14336,
              vocab 128256, random N(0, 0.02) bf16 weights): prefill of 16 x 512
              tokens and 128 greedy KV-cached decode steps; and the board's
              socket power and engine clock (amd-smi, median of samples)
              while the step runs back to back for about two seconds: these
              kernels hold the board at its power limit, which sets the clock

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
                       [--no-extra] [--no-power]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "FA2 fwd+bwd TFLOP/s & %MFMA peak; Llama-8B-shape prefill tokens/s, 1 GPU"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0

B, H, S, D = 8, 32, 4096, 128


def fwd_flops(b, hq, sq, sk, d, causal=True):
    return 4.0 * b * hq * sq * sk * d * (0.5 if causal else 1.0)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-heads", type=int, default=48,
                    help="heads of the workload the CPU baseline times")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the long-context GQA, Llama block and Llama-8B measurements")
    ap.add_argument("--no-power", action="store_true",
                    help="skip the power / clock sampling phase")
    ap.add_argument("--only", choices=["bandwidth", "block", "gqa", "gqa_short", "llama8b", "gemm"],
                    help="run only one of the secondary measurements (one JSON line): the "
                         "HBM-bound kernels at the Llama-block shapes, one Llama block, the "
                         "long-context GQA FA2, or the Llama-8B-shape prefill + decode")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="after the timed steps, run one head transpose (a pure copy) of "
                         "Q's 256 MiB, the known-size reference for HBM byte counters")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: there is no multi-GPU path (attention "
              "would shard over (batch, kv-head) with no exchange between GPUs)",
              file=sys.stderr)
        return 2

    import torch

    from teenyformers_amd import _lib, ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    _lib.lib()
    if args.only:
        run = {"bandwidth": ("bandwidth_c2", lambda: bench_bandwidth(torch, ops, _lib)),
               "block": ("llama_block", lambda: bench_llama_block(torch)),
               "gqa": ("fa2_gqa_long", lambda: bench_gqa_long(torch, ops)),
               "gqa_short": ("fa2_gqa_short", lambda: bench_gqa_short(torch, ops)),
               "llama8b": ("llama_8b_shape", lambda: bench_llama_8b(torch)),
               "gemm": ("gemm", lambda: bench_gemm(torch))}[args.only]
        print(json.dumps({run[0]: run[1]()}), flush=True)
        return 0
    gen = torch.Generator(device=dev).manual_seed(1234)
    shape = (B, H, S, D)
    q, k, v, do = (torch.randn(shape, generator=gen, device=dev).to(torch.bfloat16)
                   for _ in range(4))
    scale = 1.0 / math.sqrt(D)
    o = torch.empty_like(q)
    lse = torch.empty((B, H, S), dtype=torch.float32, device=dev)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws = torch.empty(ops.flash_attn2_bwd_workspace_bytes(q, k), dtype=torch.uint8, device=dev)

    def step():
        ops.flash_attn2_fwd(q, k, v, scale, True, out=o, lse=lse)
        ops.flash_attn2_bwd(q, k, v, o, lse, do, scale, True, workspace=ws, dq=dq, dk=dk, dv=dv)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    _lib.profile_enable(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    _lib.profile_enable(False)
    stats = _lib.profile_stats()
    if args.calibrate_copy:
        # [B, S, H*D] -> [B, H, S, D]: reads and writes q.numel() * 2 bytes
        ops.transpose_heads(q.view(B, S, H * D), H)
        torch.cuda.synchronize()

    f_fwd = fwd_flops(B, H, S, S, D)
    f_bwd = 2.5 * f_fwd
    ms_step = elapsed * 1e3 / args.steps
    value = (f_fwd + f_bwd) / (ms_step * 1e-3) / 1e12

    kernels = {}
    for name, (n, tot) in stats.items():
        kernels[name] = {"launches": n, "avg_ms": tot / max(n, 1), "total_ms": tot}
    # Algorithmic MFMA work of each kernel, in units of the forward's
    # 2 products (QK^T, PV): the dK/dV kernel does S, dP, dV, dK (2.0x fwd),
    # the dQ kernel S, dP, dQ (1.5x fwd); the backward as a whole is credited
    # the 5 products (2.5x fwd) of the FA2 convention.
    work = {"teeny_fa2_fwd_bf16": f_fwd, "teeny_fa2_bwd_dkdv_bf16": 2.0 * f_fwd,
            "teeny_fa2_bwd_dq_bf16": 1.5 * f_fwd}
    fwd_ms = sum(kernels[n]["avg_ms"] for n in kernels if n.startswith("teeny_fa2_fwd_bf16"))
    bwd_all_ms = sum(kernels[n]["avg_ms"] for n in kernels if n.startswith("teeny_fa2_bwd"))
    dominant = max((n for n in kernels if any(n.startswith(p) for p in work)),
                   key=lambda n: kernels[n]["total_ms"])
    dom_flops = next(w for p, w in work.items() if dominant.startswith(p))
    dom_ms = kernels[dominant]["avg_ms"]
    achieved = dom_flops / (dom_ms * 1e-3) / 1e12
    for name in kernels:
        kernels[name]["avg_ms"] = round(kernels[name]["avg_ms"], 4)
        kernels[name]["total_ms"] = round(kernels[name]["total_ms"], 3)

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "causal flash-attention-2 forward+backward, MHA",
                   "batch": B, "heads": H, "seq_len": S, "head_dim": D, "causal": True,
                   "flop_per_step": f_fwd + f_bwd},
        "roofline": {"bound": "mfma", "kernel": dominant,
                     "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic_from_profiles(dominant)},
        "cpu_baseline": None,
        "detail": {
            "pct_mfma_peak_step": round(value / PEAK_BF16_TFLOPS, 4),
            "fwd_tflops": round(f_fwd / (fwd_ms * 1e-3) / 1e12, 2) if fwd_ms else None,
            "fwd_pct_peak": round(f_fwd / (fwd_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)
            if fwd_ms else None,
            "bwd_tflops": round(f_bwd / (bwd_all_ms * 1e-3) / 1e12, 2) if bwd_all_ms else None,
            "bwd_pct_peak": round(f_bwd / (bwd_all_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)
            if bwd_all_ms else None,
            "kernels": kernels,
        },
    }

    if not args.no_power:
        pw = sample_power(torch, step, seconds=2.0)
        if pw is not None:
            # dense bf16 peak at the clock the board held: CUs x 4 SIMDs x 1024
            # FLOP per clock (one 32x32x16 MFMA per 32 clocks per SIMD)
            cus = torch.cuda.get_device_properties(0).multi_processor_count
            at_clk = cus * 4096 * pw["engine_clock_mhz"] * 1e6 / 1e12
            pw["peak_bf16_tflops_at_clock"] = round(at_clk, 1)
            pw["step_pct_of_clock_peak"] = round(out["value"] / at_clk, 4)
        out["detail"]["power"] = pw
    if not args.no_extra:
        del q, k, v, do, o, lse, dq, dk, dv, ws
        torch.cuda.empty_cache()
        out["detail"]["bandwidth_c2"] = bench_bandwidth(torch, ops, _lib)
        out["detail"]["fa2_gqa_long"] = bench_gqa_long(torch, ops)
        out["detail"]["fa2_gqa_short"] = bench_gqa_short(torch, ops)
        out["detail"]["gemm"] = bench_gemm(torch)
        out["detail"]["llama_block"] = bench_llama_block(torch)
        out["detail"]["llama_8b_shape"] = bench_llama_8b(torch)
        torch.cuda.empty_cache()
        gen = torch.Generator(device=dev).manual_seed(1234)
        q, k, v, do = (torch.randn(shape, generator=gen, device=dev).to(torch.bfloat16)
                       for _ in range(4))
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(q, k, v, do, scale, args.cpu_heads)
    print(json.dumps(out), flush=True)
    return 0


def _time(torch, fn, reps: int, warmup: int = 1, warm_ms: float = 60.0) -> float:
    """Mean milliseconds of fn() over reps calls (device-synchronised), after
    at least `warmup` calls and `warm_ms` of back-to-back work: the engine
    clock settles at its power limit only after some milliseconds of load,
    and a measurement that starts from idle reads up to ~15 % slow."""
    t0 = time.perf_counter()
    n = 0
    while n < warmup or (time.perf_counter() - t0) * 1e3 < warm_ms:
        fn()
        n += 1
        if n % 4 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / reps


def bench_gqa_long(torch, ops):
    """Causal GQA FA2 fwd+bwd, B1 Hq64 Hkv8 D128, S = 16384 and 8191, 1% of K
    rows scaled x8."""
    res = {}
    for S_ in (16384, 8191):
        gen = torch.Generator(device="cuda").manual_seed(S_)
        q = torch.randn((1, 64, S_, 128), generator=gen, device="cuda").to(torch.bfloat16)
        k = torch.randn((1, 8, S_, 128), generator=gen, device="cuda")
        idx = torch.randperm(S_, generator=gen, device="cuda")[: max(1, S_ // 100)]
        k[:, :, idx] *= 8
        k = k.to(torch.bfloat16)
        v = torch.randn((1, 8, S_, 128), generator=gen, device="cuda").to(torch.bfloat16)
        do = torch.randn_like(q)
        sc = 1.0 / math.sqrt(128)
        o, lse = ops.flash_attn2_fwd(q, k, v, sc, True)
        fwd_ms = _time(torch, lambda: ops.flash_attn2_fwd(q, k, v, sc, True, out=o, lse=lse), 10)
        bwd_ms = _time(torch, lambda: ops.flash_attn2_bwd(q, k, v, o, lse, do, sc, True), 10)
        f = fwd_flops(1, 64, S_, S_, 128)
        res[f"S{S_}"] = {"fwd_ms": round(fwd_ms, 3), "bwd_ms": round(bwd_ms, 3),
                         "fwd_tflops": round(f / fwd_ms / 1e9, 1),
                         "bwd_tflops": round(2.5 * f / bwd_ms / 1e9, 1),
                         "fwd_pct_peak": round(f / fwd_ms / 1e9 / PEAK_BF16_TFLOPS, 4),
                         "bwd_pct_peak": round(2.5 * f / bwd_ms / 1e9 / PEAK_BF16_TFLOPS, 4)}
        del q, k, v, do, o, lse
    return res


def bench_gqa_short(torch, ops):
    """Causal GQA FA2 at the Llama-3-8B prefill's attention shape, B16 Hq32
    Hkv8 S512 D128: forward (the prompt path) and backward, events around 20
    calls."""
    B_, Hq, Hkv, S_, D_ = 16, 32, 8, 512, 128
    gen = torch.Generator(device="cuda").manual_seed(512)
    q = torch.randn((B_, Hq, S_, D_), generator=gen, device="cuda").to(torch.bfloat16)
    k = torch.randn((B_, Hkv, S_, D_), generator=gen, device="cuda").to(torch.bfloat16)
    v = torch.randn((B_, Hkv, S_, D_), generator=gen, device="cuda").to(torch.bfloat16)
    do = torch.randn_like(q)
    sc = 1.0 / math.sqrt(D_)
    o, lse = ops.flash_attn2_fwd(q, k, v, sc, True)
    fwd_ms = _time(torch, lambda: ops.flash_attn2_fwd(q, k, v, sc, True, out=o, lse=lse), 20)
    bwd_ms = _time(torch, lambda: ops.flash_attn2_bwd(q, k, v, o, lse, do, sc, True), 20)
    f = fwd_flops(B_, Hq, S_, S_, D_)
    return {"shape": f"B{B_} Hq{Hq} Hkv{Hkv} S{S_} D{D_} causal",
            "fwd_us": round(fwd_ms * 1e3, 1), "bwd_us": round(bwd_ms * 1e3, 1),
            "fwd_tflops": round(f / fwd_ms / 1e9, 1), "bwd_tflops": round(2.5 * f / bwd_ms / 1e9, 1),
            "fwd_pct_peak": round(f / fwd_ms / 1e9 / PEAK_BF16_TFLOPS, 4),
            "bwd_pct_peak": round(2.5 * f / bwd_ms / 1e9 / PEAK_BF16_TFLOPS, 4)}


def bench_bandwidth(torch, ops, lib, reps: int = 20):
    """The HBM-bound kernels at the Llama-block shapes (B4 S2048, d2048, Hq32
    Hkv8 D64, F8192, bf16): RoPE, head transposes, RMSNorm, residual-add
    RMSNorm, SwiGLU; and the head transpose and RoPE at the attention
    benchmark's [8, 4096, 32, 128] (256 MiB), each beside a device copy of
    the same bytes.  Duration per call = HIP events (on the launch stream)
    around one replay of a graph of `reps` calls, / reps; bytes are the
    algorithmic reads + writes.  A torch device copy of Q's bytes is the
    size's practical ceiling."""
    B, S, Hq, Hkv, D, dm, F = 4, 2048, 32, 8, 64, 2048, 8192
    M = B * S
    gen = torch.Generator(device="cuda").manual_seed(7)

    def rnd(*shape):
        return torch.randn(shape, generator=gen, device="cuda").to(torch.bfloat16)

    q, k = rnd(B * Hq, S, D), rnd(B * Hkv, S, D)
    xq = rnd(B, S, Hq * D)
    x, r, w = rnd(M, dm), rnd(M, dm), rnd(dm)
    z = rnd(M, 2 * F)
    qo, ko = torch.empty_like(q), torch.empty_like(k)
    cases = [
        ("rope_fwd Q [128,2048,64]", lambda: ops.rope(q, 5e5, out=qo), 2 * q.numel() * 2),
        ("rope_fwd K [32,2048,64]", lambda: ops.rope(k, 5e5, out=ko), 2 * k.numel() * 2),
        ("transpose_heads Q [4,2048,32*64]", lambda: ops.transpose_heads(xq, Hq),
         2 * xq.numel() * 2),
        ("merge_heads O [4,32,2048,64]", lambda: ops.merge_heads(qo.view(B, Hq, S, D)),
         2 * qo.numel() * 2),
        ("rmsnorm [8192,2048]", lambda: ops.rmsnorm(x, w, 1e-5), 2 * M * dm * 2 + dm * 2 + M * 4),
        ("fused_add_rmsnorm [8192,2048]", lambda: ops.fused_add_rmsnorm(x, r, w, 1e-5),
         4 * M * dm * 2 + dm * 2 + M * 4),
        ("swiglu_fwd [8192,2*8192]", lambda: ops.swiglu(z), 3 * M * F * 2),
    ]
    qc = torch.empty_like(q)
    cases.append(("torch copy of Q's bytes (reference)", lambda: qc.copy_(q), 2 * q.numel() * 2))
    # the attention benchmark's size: [8, 4096, 32, 128] bf16, 256 MiB a tensor
    xl = rnd(8, 4096, 32 * 128)
    ql = xl.view(8 * 32, 4096, 128)
    qlo, xlc = torch.empty_like(ql), torch.empty_like(xl)
    # the Llama-3-8B-shape prefill's fused QKV split + RoPE + cache write
    qkv8 = rnd(16, 512, 48 * 128)
    q8 = torch.empty((16, 32, 512, 128), dtype=torch.bfloat16, device="cuda")
    kc8 = torch.empty((16, 8, 640, 128), dtype=torch.bfloat16, device="cuda")
    vc8 = torch.empty_like(kc8)
    cases.append(("qkv_rope_split [16,512,(32+2*8)*128]",
                  lambda: ops.qkv_rope_split(qkv8, q8, kc8, vc8, 0, 32, 8, 5e5),
                  2 * qkv8.numel() * 2))
    cases += [
        ("transpose_heads [8,4096,32*128]", lambda: ops.transpose_heads(xl, 32),
         2 * xl.numel() * 2),
        ("rope_fwd [256,4096,128]", lambda: ops.rope(ql, 5e5, out=qlo), 2 * ql.numel() * 2),
        ("torch copy of 256 MiB (reference)", lambda: xlc.copy_(xl), 2 * xl.numel() * 2),
    ]
    res = {}
    for name, fn, nbytes in cases:
        lib.profile_enable(True)  # one call recorded: which kernels it launches
        fn()
        torch.cuda.synchronize()
        lib.profile_enable(False)
        kernels = sorted(lib.profile_stats())
        # reps calls captured in one HIP graph, so the host's launch cost
        # (comparable to these ~10 us kernels) does not starve the GPU
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                fn()
        graph.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        del graph
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[name] = {"us": round(ms * 1e3, 2), "bytes": nbytes, "gbs": round(gbs, 1),
                     "pct_hbm_peak": round(gbs / PEAK_HBM_GBS, 4), "kernels": kernels}
    return res


def bench_gemm(torch, reps: int = 20):
    """bf16 y = x W^T at the prompt shapes of the Llama-3-8B shape (16 x 512
    tokens) and the Llama block (4 x 2048 tokens): this library's own GEMM
    kernel (teeny_gemm_bf16), its linear entry point (teeny_linear_bf16,
    which hands these sizes to hipBLASLt) and torch's GEMM on the same
    operands; for gate_up also the own GEMM with the SwiGLU epilogue
    (teeny_linear_swiglu_bf16) against the linear entry point followed by the
    SwiGLU kernel."""
    from teenyformers_amd import ops

    shapes = {"8b qkv": (8192, 6144, 4096), "8b o": (8192, 4096, 4096),
              "8b gate_up": (8192, 28672, 4096), "8b down": (8192, 4096, 14336),
              "block qkv": (8192, 3072, 2048), "block o": (8192, 2048, 2048),
              "block gate_up": (8192, 16384, 2048), "block down": (8192, 2048, 8192)}
    res = {}
    for name, (M, N, K) in shapes.items():
        x = torch.randn((M, K), device="cuda").to(torch.bfloat16)
        w = (0.02 * torch.randn((N, K), device="cuda")).to(torch.bfloat16)
        y = torch.empty((M, N), device="cuda", dtype=torch.bfloat16)

        def own_gemm():
            ops.call("teeny_gemm_bf16", ops._p(x), ops._p(w), ops._p(y), M, N, K, ops._stream())

        def lib_linear():
            ops.call("teeny_linear_bf16", ops._p(x), ops._p(w), ops._p(y), M, N, K, ops._stream())

        # several warm-up calls: a library's first call of a shape also
        # creates its plan and loads its kernel, longer than the warm-up time
        ms = _time(torch, own_gemm, reps, warmup=5)
        ms_l = _time(torch, lib_linear, reps, warmup=5)
        ms_t = _time(torch, lambda: torch.nn.functional.linear(x, w), reps, warmup=5)
        f = 2.0 * M * N * K
        res[name] = {"M": M, "N": N, "K": K, "ms": round(ms, 4),
                     "tflops": round(f / ms / 1e9, 1), "pct_peak": round(f / ms / 1e9 / PEAK_BF16_TFLOPS, 4),
                     "linear_tflops": round(f / ms_l / 1e9, 1),
                     "hipblaslt_tflops": round(f / ms_t / 1e9, 1),
                     "vs_hipblaslt": round(ms_t / ms, 3)}
        if "gate_up" in name:
            F = N // 2
            z = torch.empty((M, F), device="cuda", dtype=torch.bfloat16)

            def fused():
                ops.call("teeny_linear_swiglu_bf16", ops._p(x), ops._p(w), ops._p(z), M, F, K,
                         ops._stream())

            ms_f = _time(torch, fused, reps, warmup=5)
            ms_u = _time(torch, lambda: ops.swiglu(ops.linear(x, w)), reps, warmup=5)
            res[name].update({"swiglu_fused_ms": round(ms_f, 4), "linear_then_swiglu_ms": round(ms_u, 4)})
            del z
        del x, w, y
    return res


def bench_llama_block(torch):
    """One Llama block forward, B4 S2048 d2048, Hq32 Hkv8 D64, F8192, bf16."""
    from teenyformers_amd import llama

    cfg = llama.LlamaConfig(d_model=2048, n_heads=32, n_layers=1, vocab_size=32, eps=1e-5,
                            rope_base=5e5, intermediate_size=8192, n_kv_heads_=8)
    w = llama.init_weights(cfg, dtype=torch.bfloat16, seed=11)
    x = torch.randn((4, 2048, 2048), device="cuda").to(torch.bfloat16)
    ms = _time(torch, lambda: llama.block_forward(cfg, w, x), 50)
    f = llama.prefill_flops(cfg, 4, 2048) - 2.0 * 2048 * 32 * 4  # no lm_head
    return {"ms": round(ms, 3), "tflops": round(f / ms / 1e9, 1),
            "pct_peak": round(f / ms / 1e9 / PEAK_BF16_TFLOPS, 4), "flop": f}


def bench_llama_8b(torch):
    """Llama-3-8B-shaped model: prefill 16 x 512 tokens, then 128 greedy
    KV-cached decode steps (random N(0, 0.02) bf16 weights, uniform ids)."""
    from teenyformers_amd import llama, ops

    cfg = llama.LlamaConfig(d_model=4096, n_heads=32, n_layers=32, vocab_size=128256,
                            eps=1e-5, rope_base=5e5, intermediate_size=14336, n_kv_heads_=8)
    w = llama.init_weights(cfg, dtype=torch.bfloat16, seed=12)
    model = llama.Llama(cfg, w)
    Bq, Sp, n_new = 16, 512, 128
    ids = torch.randint(0, cfg.vocab_size, (Bq, Sp), device="cuda")
    cache_holder = {}

    def prefill():
        cache_holder["c"], cache_holder["l"] = model.prefill(ids, Sp + n_new)

    prefill_ms = _time(torch, prefill, 3)
    # the reference's Llama::forward (src/llama.rs:65-81) computes every
    # position's logits; the generation prefill above only the last one's
    fwd_all_ms = _time(torch, lambda: model.forward(ids), 3)
    cache, logits = cache_holder["c"], cache_holder["l"]
    nxt = ops.argmax_rows(logits).view(-1, 1)
    # decode: the decode weights in the streaming layout (a second copy, same
    # outputs), the step captured once in a HIP graph (its first run is step
    # 1), then replayed; each replay writes the next ids and one cache row
    model.stream_layout()
    dg = llama.DecodeGraph(model, cache, nxt)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(n_new - 1):
        dg.replay()
    torch.cuda.synchronize()
    decode_ms = (time.perf_counter() - t0) * 1e3 / (n_new - 1)
    f = llama.prefill_flops(cfg, Bq, Sp)
    f_all = llama.prefill_flops(cfg, Bq, Sp, last_logits_only=False)
    wbytes = sum(t.numel() * t.element_size() for t in w.values())
    del w, model, cache, dg
    return {"prefill_ms": round(prefill_ms, 2),
            "prefill_tokens_per_s": round(Bq * Sp / prefill_ms * 1e3, 1),
            "prefill_tflops": round(f / prefill_ms / 1e9, 1),
            "prefill_pct_peak": round(f / prefill_ms / 1e9 / PEAK_BF16_TFLOPS, 4),
            "prefill_logits": "last prompt position only (what generation needs)",
            "forward_all_logits_ms": round(fwd_all_ms, 2),
            "forward_all_logits_tokens_per_s": round(Bq * Sp / fwd_all_ms * 1e3, 1),
            "forward_all_logits_tflops": round(f_all / fwd_all_ms / 1e9, 1),
            "decode_ms_per_step": round(decode_ms, 3),
            "decode_tokens_per_s": round(Bq / decode_ms * 1e3, 1),
            "decode_weight_gbs": round(wbytes / decode_ms / 1e6, 1),
            "decode_pct_hbm_peak": round(wbytes / decode_ms / 1e6 / PEAK_HBM_GBS, 4),
            "decode_weights": "streaming layout (a second copy of the decode weights)",
            "decode": "one step captured in a HIP graph and replayed",
            "batch": Bq, "prompt": Sp, "new_tokens": n_new}


def _smi_sample():
    """(socket power W, mean engine clock MHz over the XCDs) from amd-smi, or None."""
    import subprocess

    try:
        r = subprocess.run(["amd-smi", "metric", "-p", "-c", "--json"], capture_output=True,
                           text=True, timeout=10)
        d = json.loads(r.stdout)["gpu_data"]
        g = d[0] if isinstance(d, list) else d
        pw = float(g["power"]["socket_power"]["value"])
        clks = [float(v["clk"]["value"]) for n, v in g["clock"].items() if n.startswith("gfx_")]
        return pw, sum(clks) / len(clks)
    except Exception:  # tool missing or output format differs: report nothing
        return None


def sample_power(torch, step, seconds: float):
    """Runs `step` back to back for `seconds` while sampling amd-smi from a
    thread; medians of the samples taken after the first half second."""
    import statistics
    import threading

    samples, stop = [], threading.Event()

    def sampler():
        t0 = time.perf_counter()
        while not stop.is_set():
            s = _smi_sample()
            if s is not None and time.perf_counter() - t0 > 0.5:
                samples.append(s)
            time.sleep(0.1)

    th = threading.Thread(target=sampler, daemon=True)
    th.start()
    t0, n = time.perf_counter(), 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            step()
        torch.cuda.synchronize()
        n += 10
    ms = (time.perf_counter() - t0) * 1e3 / n
    stop.set()
    th.join()
    if not samples:
        return None
    return {"socket_power_w": statistics.median(p for p, _ in samples),
            "engine_clock_mhz": round(statistics.median(c for _, c in samples)),
            "max_engine_clock_mhz": 2400, "samples": len(samples),
            "ms_per_step_while_sampling": round(ms, 4)}


def traffic_from_profiles(kernel: str):
    """HBM bytes per launch of `kernel` from the committed counter summaries."""
    import glob
    import re

    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*_hbm_traffic.md"))):
        with open(path) as f:
            for line in f:
                m = re.match(r"- traffic_bytes_per_launch (\S+) (\S+)", line.strip())
                if m and m.group(1) == kernel:
                    return float(m.group(2))
    return None


def cpu_baseline(q, k, v, do, scale, n_heads):
    """The oracle (the build's fp32 C restatement of the reference kernels,
    OpenMP over rows) on this host's cores.  value: the attention step's
    fwd+bwd (every key of every query row, as the reference loops) timed on
    n_heads of the 256 (b, h) heads and extrapolated linearly to all of them,
    in the same algorithmic TFLOP/s as the GPU line.  legs: the reference's
    CPU path on the other configurations, in full: the fp32 FA2 forward with
    RoPE and head transpose at B1 H4 S128 D64, and RoPE, head transpose,
    RMSNorm, residual-add RMSNorm and SwiGLU at the Llama-block shapes (fp32,
    the oracle's precision; GB/s over the fp32 bytes each moves)."""
    import numpy as np

    from oracle import oracle as O

    picks = [(i * B // n_heads, (i * 7) % H) for i in range(n_heads)]
    sel = lambda t: np.stack([t[b, h].float().cpu().numpy() for b, h in picks])[None]  # noqa
    qs, ks, vs, dos = sel(q), sel(k), sel(v), sel(do)
    threads = O.num_threads()
    t0 = time.perf_counter()
    o, lse = O.fa2_fwd(qs, ks, vs, scale, True, all_keys=True)
    t1 = time.perf_counter()
    O.fa2_bwd(qs, ks, vs, o, dos, lse, scale, True, all_keys=True)
    t2 = time.perf_counter()
    f_fwd = fwd_flops(1, n_heads, S, S, D)
    f_tot = 3.5 * f_fwd
    legs = cpu_legs(np, O)
    return {
        "value": round(f_tot / (t2 - t0) / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"fwd+bwd of {n_heads} of the {B * H} (b, h) heads at S={S}, D={D}, fp32, "
                  f"extrapolated to all {B * H} (linear in heads); fwd {t1 - t0:.2f} s, "
                  f"bwd {t2 - t1:.2f} s",
        "extrapolated": True,
        "host": _host(threads),
        "legs": legs,
    }


def cpu_legs(np, O):
    """The oracle on the other configurations, each in full (fp32)."""
    rng = np.random.default_rng(5)

    def rnd(*shape):
        return rng.standard_normal(shape, dtype=np.float32)

    def timed(fn, reps=3):
        fn()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        return (time.perf_counter() - t0) / reps

    legs = {}
    # FA2 forward, fp32, B1 H4 S128 D64: RoPE (theta 1e4) on Q and K, head
    # transpose [B,S,H,D] -> [B,H,S,D], causal attention
    Bc, Sc, Hc, Dc = 1, 128, 4, 64
    xq, xk, xv = rnd(Bc, Sc, Hc * Dc), rnd(Bc, Sc, Hc * Dc), rnd(Bc, Sc, Hc * Dc)
    lnb = float(np.log(np.float32(1e4)).astype(np.float32))

    def c1():
        qh = O.rope(O.transpose_heads(xq, Bc, Sc, Hc, Dc), lnb)
        kh = O.rope(O.transpose_heads(xk, Bc, Sc, Hc, Dc), lnb)
        vh = O.transpose_heads(xv, Bc, Sc, Hc, Dc)
        O.fa2_fwd(qh, kh, vh, 1.0 / math.sqrt(Dc), True, all_keys=True)

    sec = timed(c1, reps=20)
    f = fwd_flops(Bc, Hc, Sc, Sc, Dc)
    legs["fa2_fwd_rope_transpose B1 H4 S128 D64"] = {
        "ms": round(sec * 1e3, 3), "tflops_attention": round(f / sec / 1e12, 6)}
    # the Llama-block shapes (B4 S2048, d2048, Hq32 Hkv8 D64, F8192)
    M, dm, F = 4 * 2048, 2048, 8192
    qb = rnd(4 * 32, 2048, 64)
    xb = rnd(4, 2048, 32 * 64)
    x, r, w = rnd(M, dm), rnd(M, dm), rnd(dm)
    z = rnd(M, 2 * F)
    lnb5 = float(np.log(np.float32(5e5)).astype(np.float32))
    cases = [
        ("rope_fwd Q [128,2048,64]", lambda: O.rope(qb, lnb5), 2 * qb.size * 4),
        ("transpose_heads Q [4,2048,32*64]", lambda: O.transpose_heads(xb, 4, 2048, 32, 64),
         2 * xb.size * 4),
        ("rmsnorm [8192,2048]", lambda: O.rmsnorm_fwd(x, w, 1e-5), 2 * M * dm * 4),
        ("fused_add_rmsnorm [8192,2048]", lambda: O.fused_add_rmsnorm_fwd(x, r, w, 1e-5),
         4 * M * dm * 4),
        ("swiglu_fwd [8192,2*8192]", lambda: O.swiglu_fwd(z), 3 * M * F * 4),
    ]
    for name, fn, nbytes in cases:
        sec = timed(fn)
        legs[name] = {"ms": round(sec * 1e3, 3), "gbs": round(nbytes / sec / 1e9, 2)}
    return legs


def _host(threads):
    """This host: CPU model, logical CPUs, the CPUs this process may use."""
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = None
    return {"cpu": _cpu_model(), "nproc": os.cpu_count(), "usable_cpus": usable,
            "oracle_threads": threads}


def _cpu_model():
    """The CPU model string: lscpu's "Model name" (with its vendor and family
    fields when the name alone is generic), else /proc/cpuinfo."""
    import subprocess

    fields = {}
    try:
        r = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10)
        for line in r.stdout.splitlines():
            if ":" in line:
                key, val = line.split(":", 1)
                fields[key.strip()] = val.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    name = fields.get("Model name")
    if not name:
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("model name"):
                        name = line.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
    extra = [f"{k} {fields[k]}" for k in ("Vendor ID", "CPU family", "Model", "Socket(s)",
                                          "Core(s) per socket", "Thread(s) per core")
             if k in fields]
    return "; ".join([name or "unknown"] + extra)


if __name__ == "__main__":
    sys.exit(main())

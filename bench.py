#!/usr/bin/env python3
"""Benchmark of the bfp16 prefill MUL_MAT path on one MI355X.

Workload (the north star's target): the Qwen3-4B-shaped
36-layer decoder stack, random-init Q4_K (Q/K/V/gate/up) and Q8_0 (O/down)
weights converted once into the resident bfp16 cache, an 8192-token fp32
N(0,1) prompt processed in 2048-token chunks: per layer RMSNorm -> packed
Q/K/V GEMMs, O GEMM + residual, RMSNorm -> one fused gate/up GEMM whose
epilogue computes the SwiGLU and packs it -> down GEMM + residual. Attention is excluded, as BASELINE states. One step =
one whole prompt (4 chunks x 36 layers); inputs resident in HBM.

Prints one JSON line: value = MUL_MAT TFLOP/s of the whole step (matmul FLOPs
over wall time, packs and fused host ops included), with tok/s, the GEMM
kernel's roofline from HIP events around every GEMM launch of the timed
steps, and the reference's CPU path (the xdna-ref loop restated in
oracle/, built with the reference's flags) on a bounded sample.

    python bench.py [--steps K] [--warmup W] [--workload qwen3-4b] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
METRIC = "bfp16 prefill MUL_MAT TFLOP/s (% bf16 MFMA peak); layer-stack prefill tok/s"
BF16_PEAK = 2516.6   # TFLOP/s, MI355X dense bf16 MFMA
HBM_PEAK = 8000.0    # GB/s


def load_pkg():
    sys.path.insert(0, str(ROOT))
    from __graft_entry__ import _import_pkg
    return _import_pkg()


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(cfg, tokens: int) -> dict:
    """The reference's CPU matmul (src/xdna-ref.cpp:10-97, restated in
    oracle/zest_oracle.c, built with -O3 -mavx2 -mfma -ffast-math as
    CMakeLists.txt:117) on one layer's seven matmuls at `tokens` tokens;
    threads = the cores this process may use, capped at the box's share."""
    import numpy as np
    import torch
    sys.path.insert(0, str(ROOT / "tests"))
    from helpers import Oracle  # CPU baseline leg only
    from ggml_xdna_amd import quant

    orc = Oracle(fast=True)
    threads = min(len(os.sched_getaffinity(0)), 16)
    g = torch.Generator().manual_seed(1)
    flops, secs = 0.0, 0.0
    for name, n, k, t in cfg.matmuls():
        w = torch.randn((n, k), generator=g) * 0.02
        raw = quant.quantize(t, w).numpy()
        x = torch.randn((tokens, k), generator=g).numpy()
        y = np.empty((tokens, n), dtype=np.float32)
        t0 = time.perf_counter()
        orc.L.orc_ref_mul_mat(t, raw.ctypes.data_as(orc_p()), n, k, x.ctypes.data_as(orc_p()), tokens,
                              y.ctypes.data_as(orc_p()), threads)
        secs += time.perf_counter() - t0
        flops += 2.0 * tokens * n * k
    per_token_layer = secs / tokens
    return {
        "value": round(flops / secs / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
        "sample": f"one {cfg.name} layer's 7 matmuls at {tokens} tokens ({flops / 1e9:.0f} GFLOP, {secs:.1f} s); "
                  f"tok/s for the {cfg.layers}-layer stack extrapolated from per-shape timings",
        "tok_per_s": round(1.0 / (per_token_layer * cfg.layers), 3),
        "cpu_model": cpu_model(), "affinity_cpus": len(os.sched_getaffinity(0)),
    }


def orc_p():
    import ctypes
    return ctypes.c_void_p


def pack_bandwidth(z, m: int, k: int, reps: int = 20) -> list:
    """The activation pack, as bfp16 bytes (4 + 1.125 B/value) and as the
    GEMM's expanded operand (4 + 2 B/value, the form the stack uses)."""
    import torch
    x = torch.randn((m, k), device="cuda")
    res = []
    for name, fn, out, per in (("bfp16", z.pack_act, z.empty_packed(m, k), 5.125),
                               ("expanded", z.pack_act_x, z.empty_act(m, k), 6.0)):
        fn(x, out=out)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn(x, out=out)
        e1.record()
        e1.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        gbs = per * m * k / (us * 1e-6) / 1e9
        res.append({"output": name, "shape": [m, k], "us": round(us, 2), "GB/s": round(gbs, 1),
                    "frac": round(gbs / HBM_PEAK, 3)})
    return res


def convert_bandwidth(z, wtype: int, n: int, k: int, reps: int = 10) -> dict:
    """One-time weight conversion of one [n][k] GGUF weight, repeated."""
    import torch
    from ggml_xdna_amd import quant
    raw = quant.quantize(wtype, torch.randn((n, k), device="cuda") * 0.02)
    out = z.empty_packed(n, k)
    z.convert_weight(wtype, raw, n, k, out=out)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        z.convert_weight(wtype, raw, n, k, out=out)
    e1.record()
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    nbytes = raw.numel() + n * k * 9 / 8
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"type": {8: "Q8_0", 12: "Q4_K"}[wtype], "shape": [n, k], "us": round(us, 2), "GB/s": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK, 3)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="qwen3-4b")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-tokens", type=int, default=2048)
    ap.add_argument("--unfused", action="store_true", help="gate and up as two GEMMs plus a SwiGLU kernel")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        return 2

    import torch
    z = load_pkg()
    from ggml_xdna_amd.stack import CONFIGS, Stack

    torch.cuda.set_device(0)
    z.init(0)
    z.self_test()
    cfg = CONFIGS[args.workload]
    t_build = time.perf_counter()
    stack = Stack(cfg, seed=0, fused=not args.unfused)
    torch.cuda.synchronize()
    print(f"[bench] {cfg.name}: weights converted in {time.perf_counter() - t_build:.1f} s "
          f"(kernel time {stack.convert_ms:.1f} ms)", file=sys.stderr, flush=True)

    for _ in range(args.warmup):
        stack.run_prompt()
    torch.cuda.synchronize()

    events: list = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        stack.run_prompt(gemm_events=events)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / args.steps

    flops_step = cfg.flops_per_token() * cfg.tokens
    value = flops_step / (ms_step * 1e-3) / 1e12
    gemm_ms = sum(a.elapsed_time(b) for a, b, _ in events)
    gemm_flops = sum(f for _, _, f in events)
    achieved = gemm_flops / (gemm_ms * 1e-3) / 1e12
    print(f"[bench] {args.steps} steps: {ms_step:.2f} ms/step, GEMM {gemm_ms / args.steps:.2f} ms/step over "
          f"{len(events) // args.steps} launches", file=sys.stderr, flush=True)

    pack = pack_bandwidth(z, cfg.chunk, cfg.q)
    convert = [convert_bandwidth(z, cfg.ffn_type, cfg.ffn, cfg.hidden),
               convert_bandwidth(z, cfg.down_type, cfg.hidden, cfg.ffn)]
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"{cfg.name} stack: {cfg.layers} layers, hidden {cfg.hidden}, {cfg.tokens}-token "
                               f"prompt in {cfg.chunk}-token chunks, random-init GGUF weights, attention excluded",
                   "tokens": cfg.tokens, "chunk": cfg.chunk, "layers": cfg.layers,
                   "gate_up": "two GEMMs + SwiGLU kernel" if args.unfused else
                              "one fused GEMM, SwiGLU and pack in its epilogue",
                   "operands": "bfp16 (8-value blocks, shared exponent, int8 mantissas) expanded to bf16 for "
                               "MFMA, fp32 accumulate and output"},
        "pct_bf16_peak": round(100 * value / BF16_PEAK, 2),
        "tok_per_s": round(cfg.tokens / (ms_step * 1e-3), 1),
        "roofline": {"bound": "mfma", "kernel": "gemm_kernel", "achieved": round(achieved, 2), "peak": BF16_PEAK,
                     "unit": "TFLOP/s", "frac": round(achieved / BF16_PEAK, 4), "traffic": None,
                     "launches": len(events), "avg_launch_us": round(gemm_ms * 1e3 / len(events), 2)},
        "convert": convert,
        "pack": pack,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(cfg, args.cpu_tokens)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

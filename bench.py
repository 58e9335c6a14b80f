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
kernel's roofline (the step's GEMM launches run back to back between two HIP
events: the same shapes, tiles and K splits), and the reference's CPU path
(the xdna-ref loop restated in oracle/, built with the reference's flags) on
a bounded sample.

    python bench.py [--steps K] [--warmup W] [--workload qwen3-4b] [--chunk M] [--no-cpu]
    python bench.py --hbm      # converter (every GGUF type) and pack HBM rates
    python bench.py --kernel-configs   # BASELINE configs 1 and 2, launch by launch

The roofline's `traffic` (HBM bytes per GEMM launch) comes from two
rocprofv3 counter runs of this script's probe mode, summarised into
profiles/gemm_traffic_<workload>.json:

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d <dir_f> -o run -- python3 bench.py --traffic-probe
    rocprofv3 --pmc WRITE_SIZE --output-format csv -d <dir_w> -o run -- python3 bench.py --traffic-probe
    python3 bench.py --traffic-summary <dir_f> <dir_w> > profiles/gemm_traffic_qwen3-4b.json

The probe runs one prompt step, then a calibration kernel of known traffic
(zest_scale over 64 Mi floats: 256 MiB read, 256 MiB written); each counter
is scaled by what it reads for that kernel.
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
BOARD_POWER_LIMIT_W = 1400  # MI355X total board power, as published


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


# GGUF block types: (values per block, bytes per block, byte ranges of the
# block's fp16 scale fields)
GGUF_BLOCKS = {"F16": (1, 1, 2, []), "BF16": (30, 1, 2, []), "Q4_0": (2, 32, 18, [(0, 2)]),
               "Q4_1": (3, 32, 20, [(0, 4)]), "Q5_0": (6, 32, 22, [(0, 2)]), "Q5_1": (7, 32, 24, [(0, 4)]),
               "Q8_0": (8, 32, 34, [(0, 2)]), "Q2_K": (10, 256, 84, [(80, 84)]), "Q3_K": (11, 256, 110, [(108, 110)]),
               "Q4_K": (12, 256, 144, [(0, 4)]), "Q5_K": (13, 256, 176, [(0, 4)]), "Q6_K": (14, 256, 210, [(208, 210)]),
               "IQ4_NL": (20, 32, 18, [(0, 2)]), "IQ4_XS": (23, 256, 136, [(0, 2)])}


def random_gguf(name: str, n: int, k: int, seed: int):
    """n rows of random GGUF blocks with finite scales (the converter's speed
    does not depend on the values)."""
    import torch
    wtype, blk, bb, fields = GGUF_BLOCKS[name]
    g = torch.Generator(device="cuda").manual_seed(seed)
    raw = torch.randint(0, 256, (n * (k // blk), bb), dtype=torch.uint8, device="cuda", generator=g)
    if blk == 1:  # F16 / BF16: keep the exponent field off all-ones
        v = raw.view(-1).view(torch.int16)
        top = 0x7C00 if wtype == 1 else 0x7F80
        v[(v & top) == top] &= 0x3FFF
    for lo, hi in fields:
        d = (torch.rand((raw.shape[0], (hi - lo) // 2), device="cuda", generator=g) * 0.01).to(torch.float16)
        raw[:, lo:hi] = d.view(torch.uint8)
    return raw.view(n, -1)


# The HBM-rate measurements: every launch takes the next of several input and
# output sets, at least 4 and enough that their footprint is three times the
# 256 MB MALL, so each launch reads its input from HBM rather than from the
# cache the previous launch filled.
HBM_REPS = 5
HBM_W = (17408, 5120)  # converter: one weight of the 27B-class FFN
HBM_X = (8192, 5120)   # pack and RMSNorm: 8192 activation rows of 5120


def _sets(set_bytes: float) -> int:
    return max(4, int(768e6 // set_bytes) + 1)


def _timed(fn, count: int) -> float:
    """Average microseconds per call over `count` calls after one warm call,
    between HIP events on the current stream."""
    import torch
    fn(0)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(count):
        fn(i)
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e3 / count


def _rate(kernel: str, nbytes: float, us: float, **kw) -> dict:
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"kernel": kernel, **kw, "bytes": int(nbytes), "us": round(us, 2), "GB/s": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK, 3)}


def convert_rate(z, name: str, n: int = HBM_W[0], k: int = HBM_W[1]) -> dict:
    """One-time weight conversion of an [n][k] GGUF weight of type `name`:
    GGUF bytes read + 1.125 B/value written."""
    wtype, blk, bb, _ = GGUF_BLOCKS[name]
    nbytes = n * (k // blk) * bb + n * k * 9 / 8
    sets = _sets(nbytes)
    raws = [random_gguf(name, n, k, s) for s in range(sets)]
    outs = [z.empty_packed(n, k) for _ in range(sets)]
    us = _timed(lambda i: z.convert_weight(wtype, raws[i % sets], n, k, out=outs[i % sets]), sets * HBM_REPS)
    return _rate("convert", nbytes, us, type=name, shape=[n, k])


def pack_rates(z, m: int = HBM_X[0], k: int = HBM_X[1], bfp16: bool = True) -> list:
    """The activation pack, to bfp16 bytes (4 + 1.125 B/value) and to the
    GEMM's expanded operand (4 + 2 B/value, the form the stack uses)."""
    import torch
    sets = _sets(6.0 * m * k)
    xs = [torch.randn((m, k), device="cuda") for _ in range(sets)]
    res = []
    for label, fn, mk, per in (("pack", z.pack_act, z.empty_packed, 5.125), ("pack_x", z.pack_act_x, z.empty_act, 6.0)):
        if label == "pack" and not bfp16:
            continue
        outs = [mk(m, k) for _ in range(sets)]
        us = _timed(lambda i: fn(xs[i % sets], out=outs[i % sets]), sets * HBM_REPS)
        res.append(_rate(label, per * m * k, us, shape=[m, k]))
        del outs
    return res


def norm_rate(z, m: int = HBM_X[0], d: int = HBM_X[1]) -> dict:
    """RMSNorm with its scale row, writing only the next matmul's expanded
    operand (the stack's form): 4 + 2 B/value."""
    import torch
    sets = _sets(6.0 * m * d)
    xs = [torch.randn((m, d), device="cuda") for _ in range(sets)]
    w = torch.randn(d, device="cuda")
    outs = [z.empty_act(m, d) for _ in range(sets)]
    us = _timed(lambda i: z.rms_norm(xs[i % sets], 1e-6, w, y=None, packed=outs[i % sets]), sets * HBM_REPS)
    return _rate("rms_norm+pack_x", 6.0 * m * d, us, shape=[m, d])


def copy_rate(nbytes: float) -> dict:
    """The ceiling the HBM-bound kernels are held against: torch's device
    copy of a float32 tensor, `nbytes` moved in all (half read, half
    written), on rotating sets as above."""
    import torch
    n = int(nbytes / 8)
    sets = _sets(nbytes)
    xs = [torch.randn(n, device="cuda") for _ in range(sets)]
    ys = [torch.empty_like(xs[0]) for _ in range(sets)]
    us = _timed(lambda i: ys[i % sets].copy_(xs[i % sets]), sets * HBM_REPS)
    return _rate("copy", 8.0 * n, us, floats=n)


def hbm_kernels(args) -> int:
    """HBM rates of the converter (every GGUF type), the activation pack and
    the fused RMSNorm+pack, on rotating sets, at the large shapes and at the
    qwen3-4b stack's own, beside a plain copy of the same bytes. One JSON
    line per kernel."""
    import torch
    z = load_pkg()
    torch.cuda.set_device(0)
    z.init(0)
    for name in GGUF_BLOCKS:
        print(json.dumps(convert_rate(z, name)), flush=True)
    for r in pack_rates(z):
        print(json.dumps(r), flush=True)
    print(json.dumps(norm_rate(z)), flush=True)
    # the stack's own sizes: qwen3-4b's attention output (2048 x 4096) and hidden rows (2048 x 2560)
    for r in pack_rates(z, 2048, 4096, bfp16=False):
        print(json.dumps(r), flush=True)
    print(json.dumps(norm_rate(z, 2048, 2560)), flush=True)
    # a plain copy moving the same bytes as each of the above
    for nbytes in (6.0 * 2048 * 2560, 6.0 * 2048 * 4096, 6.0 * HBM_X[0] * HBM_X[1],
                   HBM_W[0] * HBM_W[1] * (34 / 32 + 9 / 8)):
        print(json.dumps(copy_rate(nbytes)), flush=True)
    return 0


def operand_activity(args) -> int:
    """The same GEMM launches on operands of different bit activity: random
    bytes, the workload's own kind (N(0,1) activations against quantised
    N(0, 0.02) Q4_K weights), and operands whose mantissas are all zero (the
    matrix core's inputs then do not toggle). The kernel, shapes, tiles and
    memory traffic are the same in every case; only the data's switching
    activity, and so the chip's power draw and clock, differ. One JSON line
    per shape, microseconds and TFLOP/s per case."""
    import torch
    z = load_pkg()
    import ggml_xdna_amd.quant as quant
    torch.cuda.set_device(0)
    z.init(0)
    for (m, n, k) in ACTIVITY_SHAPES:
        g = torch.Generator(device="cuda").manual_seed(0)
        a_x = z.pack_act_x(torch.randn((m, k), device="cuda", generator=g))
        a_zero = z.pack_act_x(torch.zeros((m, k), device="cuda"))
        w_rand = torch.randint(0, 256, (z.bfp16_bytes(n, k),), dtype=torch.uint8, device="cuda", generator=g)
        tiles = w_rand.view(-1, 1152)
        tiles[:, 1024:] = torch.randint(118, 128, (tiles.shape[0], 128), dtype=torch.uint8, device="cuda", generator=g)
        w_q4k = z.convert_weight(12, quant.quantize(12, torch.randn((n, k), device="cuda", generator=g) * 0.02), n, k)
        w_zero = w_rand.clone()
        w_zero.view(-1, 1152)[:, :1024] = 0  # mantissas zero, exponent bytes kept
        c = torch.empty((m, n), device="cuda")
        res = {}
        operands = {"random bytes": (a_x, w_rand), "workload data": (a_x, w_q4k), "W mantissas zero": (a_x, w_zero),
                    "A zero": (a_zero, w_q4k), "workload data again": (a_x, w_q4k)}
        for name in ACTIVITY_CASES:
            a, w = operands[name]
            us = _timed(lambda i: z.gemm(a, m, w, n, k, out=c), activity_reps(m, n, k))
            res[name] = {"us": round(us, 1), "TFLOP/s": round(2.0 * m * n * k / us / 1e6, 1)}
        print(json.dumps({"shape": [m, n, k], "cases": res}), flush=True)
    return 0


def kernel_configs(args) -> int:
    """BASELINE configs[0] and [1] on one GPU, inputs and converted weights
    resident, HIP events around back-to-back repetitions after one warm call:
    config 1, one MUL_MAT 1024 x 2560 x 2560 with a Q8_0 weight (the
    activation pack, then the GEMM); config 2, the SwiGLU FFN triple at 2048
    tokens with 1% of the K-channels scaled x20 and Q4_K weights (the pack, the
    fused gate/up GEMM that computes the SwiGLU and packs it in its epilogue,
    the down GEMM). One JSON line per config: each launch alone, the chain back
    to back, TFLOP/s and % of the bf16 peak, and the weights' one-time
    conversion."""
    import torch
    z = load_pkg()
    import ggml_xdna_amd.quant as quant
    torch.cuda.set_device(0)
    z.init(0)
    g = torch.Generator(device="cuda").manual_seed(0)

    def tf(flops, us):
        return {"us": round(us, 2), "TFLOP/s": round(flops / us / 1e6, 1), "pct_peak": round(flops / us / 1e6 / BF16_PEAK * 100, 2)}

    # config 1
    M, N, K = 1024, 2560, 2560
    x = torch.randn((M, K), device="cuda", generator=g)
    raw = quant.quantize(8, torch.randn((N, K), device="cuda", generator=g) * 0.02)
    w = z.empty_packed(N, K)
    conv = _timed(lambda i: z.convert_weight(8, raw, N, K, out=w), 20)
    a = z.empty_act(M, K)
    c = torch.empty((M, N), device="cuda")
    fl = 2.0 * M * N * K
    pack = _timed(lambda i: z.pack_act_x(x, out=a), KCONFIG_REPS)
    gemm = _timed(lambda i: z.gemm(a, M, w, N, K, out=c), KCONFIG_REPS)
    both = _timed(lambda i: (z.pack_act_x(x, out=a), z.gemm(a, M, w, N, K, out=c)), KCONFIG_REPS)
    print(json.dumps({"config": 1, "shape": [M, N, K], "weight": "Q8_0", "gemm": tf(fl, gemm),
                      "pack_us": round(pack, 2), "pack_and_gemm": tf(fl, both), "convert_us": round(conv, 2)}), flush=True)

    # config 2
    M, D, F = 2048, 2560, 9728
    x = torch.randn((M, D), device="cuda", generator=g)
    ch = torch.randperm(D, generator=g, device="cuda")[: D // 100]
    x[:, ch] *= 20.0
    gate, up, down = (quant.quantize(12, torch.randn(shape, device="cuda", generator=g) * 0.02)
                      for shape in ((F, D), (F, D), (D, F)))
    wgu, wd = z.empty_packed(2 * F, D), z.empty_packed(D, F)
    conv_gu = _timed(lambda i: z.convert_weight_gu(12, gate, up, F, D, out=wgu), 10)
    conv_d = _timed(lambda i: z.convert_weight(12, down, D, F, out=wd), 10)
    a, h = z.empty_act(M, D), z.empty_act(M, F)
    y = torch.empty((M, D), device="cuda")
    fl_gu, fl_d = 4.0 * M * F * D, 2.0 * M * D * F
    pack = _timed(lambda i: z.pack_act_x(x, out=a), KCONFIG_REPS)
    glu = _timed(lambda i: z.gemm_glu(z.GLU_SWIGLU, a, M, wgu, F, D, xout=h), KCONFIG_REPS)
    dn = _timed(lambda i: z.gemm(h, M, wd, D, F, out=y), KCONFIG_REPS)
    chain = _timed(lambda i: (z.pack_act_x(x, out=a), z.gemm_glu(z.GLU_SWIGLU, a, M, wgu, F, D, xout=h),
                              z.gemm(h, M, wd, D, F, out=y)), KCONFIG_REPS)
    print(json.dumps({"config": 2, "tokens": M, "hidden": D, "ffn": F, "weight": "Q4_K", "outliers": "1% of K x20",
                      "gate_up_glu": tf(fl_gu, glu), "down": tf(fl_d, dn), "pack_us": round(pack, 2),
                      "triple": tf(fl_gu + fl_d, chain), "convert_gate_up_us": round(conv_gu, 2),
                      "convert_down_us": round(conv_d, 2)}), flush=True)
    return 0


KCONFIG_REPS = 50

ACTIVITY_SHAPES = ((8192, 8192, 8192), (2048, 19456, 2560), (2048, 2560, 9728))
ACTIVITY_CASES = ("random bytes", "workload data", "W mantissas zero", "A zero", "workload data again")


def activity_reps(m: int, n: int, k: int) -> int:
    return 10 if m * n * k > 2e11 else 40


def activity_summary(pmc_dir: str, trace_dir: str) -> int:
    """Per shape and case of --operand-activity under rocprofv3: the GEMM's
    average duration (kernel trace), its clock (GRBM_GUI_ACTIVE, summed over
    the 8 XCDs, over the duration) and the MFMA-busy share of the SIMD cycles
    (SQ_VALU_MFMA_BUSY_CYCLES), over each case's timed launches."""
    import csv
    import glob
    from collections import defaultdict
    per = defaultdict(float)
    for r in _counter_rows(pmc_dir):
        if "gemm_kernel" in r["Kernel_Name"]:
            per[(int(r["Dispatch_Id"]), r["Counter_Name"])] += float(r["Counter_Value"])
    ids = sorted({d for d, _ in per})
    durs = []
    for f in glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True):
        rows = sorted(csv.DictReader(open(f)), key=lambda r: int(r["Start_Timestamp"]))
        durs += [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3 for r in rows
                 if "gemm_kernel" in r["Kernel_Name"]]
    sizes = [1 + activity_reps(*sh) for sh in ACTIVITY_SHAPES for _ in ACTIVITY_CASES]
    if len(ids) != sum(sizes) or len(durs) != sum(sizes):
        print(f"expected {sum(sizes)} GEMM dispatches, found {len(ids)} counted and {len(durs)} traced",
              file=sys.stderr)
        return 1
    out, at = [], 0
    for sh in ACTIVITY_SHAPES:
        m, n, k = sh
        for case in ACTIVITY_CASES:
            sel = range(at + 1, at + 1 + activity_reps(*sh))  # the warm launch left out
            at += 1 + activity_reps(*sh)
            us = sum(durs[i] for i in sel) / len(sel)
            xcd = sum(per[(ids[i], "GRBM_GUI_ACTIVE")] for i in sel) / len(sel) / 8.0
            busy = sum(per[(ids[i], "SQ_VALU_MFMA_BUSY_CYCLES")] for i in sel) / len(sel)
            out.append({"shape": list(sh), "case": case, "us": round(us, 1),
                        "TFLOP/s": round(2.0 * m * n * k / us / 1e6, 1), "clock_ghz": round(xcd / (us * 1e3), 3),
                        "mfma_busy_pct": round(100.0 * busy / (xcd * 1024), 1)})
    print(json.dumps(out, indent=1))
    return 0


SUSTAIN_SHAPE = (2048, 19456, 2560)  # the fused gate/up's GEMM at 2048 tokens, as a plain launch
SUSTAIN_CASES = ("workload data", "W mantissas zero", "random bytes")


def sustain_kinds(args) -> int:
    """The qwen3-4b stack's four GEMM launch kinds at 2048 tokens (the q/k/v
    group, O + residual, the fused gate/up with its SwiGLU, down + residual),
    each back to back for `args.sustain_kinds` seconds on the workload's kind
    of data after two idle seconds, for sampling the board's power and clock
    beside it. One JSON line per phase, as --sustain prints them."""
    import time
    import torch
    z = load_pkg()
    import ggml_xdna_amd.quant as quant
    torch.cuda.set_device(0)
    z.init(0)
    g = torch.Generator(device="cuda").manual_seed(0)
    M, H, Q, KV, F = 2048, 2560, 4096, 1024, 9728

    def weight(t, n, k):
        return z.convert_weight(t, quant.quantize(t, torch.randn((n, k), device="cuda", generator=g) * 0.02), n, k)

    a, ao, ad = (z.pack_act_x(torch.randn((M, k), device="cuda", generator=g)) for k in (H, Q, F))
    wq, wk, wv, wo, wd = weight(12, Q, H), weight(12, KV, H), weight(12, KV, H), weight(8, H, Q), weight(8, H, F)
    gate, up = (quant.quantize(12, torch.randn((F, H), device="cuda", generator=g) * 0.02) for _ in range(2))
    wgu = z.convert_weight_gu(12, gate, up, F, H)
    qo, ko, vo = torch.empty((M, Q), device="cuda"), torch.empty((M, KV), device="cuda"), torch.empty((M, KV), device="cuda")
    h = torch.randn((M, H), device="cuda", generator=g)
    xo = z.empty_act(M, F)
    kinds = {
        "qkv": (lambda: z.gemm_group(a, M, [wq, wk, wv], [Q, KV, KV], H, outs=[qo, ko, vo]), 2.0 * M * (Q + 2 * KV) * H),
        "o": (lambda: z.gemm_residual(ao, M, wo, H, Q, h, out=h), 2.0 * M * H * Q),
        "gate_up": (lambda: z.gemm_glu(z.GLU_SWIGLU, a, M, wgu, F, H, xout=xo), 4.0 * M * F * H),
        "down": (lambda: z.gemm_residual(ad, M, wd, H, F, h, out=h), 2.0 * M * H * F),
    }
    for name, (fn, flops) in kinds.items():
        torch.cuda.synchronize()
        t = time.time()
        time.sleep(2.0)
        print(json.dumps({"phase": "idle", "t0": t, "t1": time.time()}), flush=True)
        t0, launches = time.time(), 0
        while time.time() - t0 < args.sustain_kinds:
            for _ in range(20):
                fn()
            launches += 20
            torch.cuda.synchronize()
        t1 = time.time()
        print(json.dumps({"phase": name, "t0": t0, "t1": t1, "launches": launches,
                          "TFLOP/s": round(flops * launches / (t1 - t0) / 1e12, 1)}), flush=True)
    return 0


def sustain(args) -> int:
    """The same GEMM launch, back to back for `args.sustain` seconds per
    operand case (the cases of --operand-activity), each after two idle
    seconds, for sampling the board's power and clock beside it (amd-smi
    from another process). One JSON line per phase: its wall-clock start and
    end (time.time()) and its TFLOP/s."""
    import time
    import torch
    z = load_pkg()
    import ggml_xdna_amd.quant as quant
    torch.cuda.set_device(0)
    z.init(0)
    m, n, k = SUSTAIN_SHAPE
    g = torch.Generator(device="cuda").manual_seed(0)
    a = z.pack_act_x(torch.randn((m, k), device="cuda", generator=g))
    w_rand = torch.randint(0, 256, (z.bfp16_bytes(n, k),), dtype=torch.uint8, device="cuda", generator=g)
    w_rand.view(-1, 1152)[:, 1024:] = torch.randint(118, 128, (w_rand.numel() // 1152, 128), dtype=torch.uint8,
                                                      device="cuda", generator=g)
    w_q4k = z.convert_weight(12, quant.quantize(12, torch.randn((n, k), device="cuda", generator=g) * 0.02), n, k)
    w_zero = w_q4k.clone()
    w_zero.view(-1, 1152)[:, :1024] = 0
    c = torch.empty((m, n), device="cuda")
    weights = {"workload data": w_q4k, "W mantissas zero": w_zero, "random bytes": w_rand}
    for case in SUSTAIN_CASES:
        torch.cuda.synchronize()
        t = time.time()
        time.sleep(2.0)
        print(json.dumps({"phase": "idle", "t0": t, "t1": time.time()}), flush=True)
        w = weights[case]
        t0, launches = time.time(), 0
        while time.time() - t0 < args.sustain:
            for _ in range(20):
                z.gemm(a, m, w, n, k, out=c)
            launches += 20
            torch.cuda.synchronize()
        t1 = time.time()
        print(json.dumps({"phase": case, "t0": t0, "t1": t1, "launches": launches,
                          "TFLOP/s": round(2.0 * m * n * k * launches / (t1 - t0) / 1e12, 1)}), flush=True)
    return 0


def _flat(d, prefix=""):
    out = {}
    for key, v in (d.items() if isinstance(d, dict) else enumerate(d)):
        name = f"{prefix}.{key}" if prefix else str(key)
        if isinstance(v, (dict, list)):
            out.update(_flat(v, name))
        else:
            out[name] = v
    return out


def sustain_summary(phases_log: str, smi_log: str) -> int:
    """Per phase of --sustain: the averages of amd-smi's samples taken inside
    it (its first second left out), from a log of lines "T <time.time()>"
    each followed by the JSON of `amd-smi metric -g 0 -p -c --json`: socket
    power and the GFX clock (the mean over the XCDs' clocks)."""
    phases = [json.loads(l) for l in open(phases_log) if l.startswith("{")]
    samples, t, buf = [], None, []

    def flush():
        if t is not None and buf:
            try:
                samples.append((t, _flat(json.loads("".join(buf)))))
            except ValueError:
                pass

    for line in open(smi_log):
        if line.startswith("T "):
            flush()
            t, buf = float(line.split()[1]), []
        else:
            buf.append(line)
    flush()
    out = []
    for ph in phases:
        inside = [f for (ts, f) in samples if ph["t0"] + 1.0 <= ts <= ph["t1"]]
        row = {"phase": ph["phase"], "samples": len(inside)}
        if "TFLOP/s" in ph:
            row["TFLOP/s"] = ph["TFLOP/s"]
        for label, pick in (("socket_power_W", lambda key: key.endswith("power.socket_power.value")),
                            ("gfx_clock_mhz", lambda key: ".clock.gfx_" in key and key.endswith(".clk.value"))):
            vals = [float(v) for f in inside for key, v in f.items() if pick(key) and str(v).replace(".", "").isdigit()]
            row[label] = round(sum(vals) / len(vals), 1) if vals else None
        out.append(row)
    print(json.dumps(out, indent=1))
    return 0


CALIB_FLOATS = 64 << 20  # the calibration kernel's floats: 256 MiB each way


def traffic_probe(args) -> int:
    """One prompt step of the workload, then the calibration kernel."""
    import torch
    z = load_pkg()
    from ggml_xdna_amd.stack import CONFIGS, Stack
    torch.cuda.set_device(0)
    z.init(0)
    cfg = CONFIGS[args.workload]
    stack = Stack(cfg, seed=0, chunk=args.chunk)
    stack.run_prompt()
    torch.cuda.synchronize()
    x = torch.randn(CALIB_FLOATS, device="cuda")
    y = torch.empty_like(x)
    z.scale(x, 1.0, 0.0, y=y)
    torch.cuda.synchronize()
    print(f"[probe] {cfg.name}: one step and the calibration kernel done", flush=True)
    return 0


def _counter_rows(d: str):
    import csv
    import glob
    for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        yield from csv.DictReader(open(f))


def traffic_summary(fetch_dir: str, write_dir: str) -> int:
    """Average FETCH_SIZE and WRITE_SIZE (KiB per dispatch) of the GEMM
    launches, each scaled by the calibration kernel's reading."""
    res = {}
    for counter, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        gemm, calib = [], []
        for r in _counter_rows(d):
            if r.get("Counter_Name") != counter:
                continue
            v = float(r["Counter_Value"]) * 1024.0  # KiB -> bytes
            if "gemm_kernel" in r["Kernel_Name"]:
                gemm.append(v)
            elif "scale_kernel" in r["Kernel_Name"]:
                calib.append(v)
        if not gemm or not calib:
            print(f"no {counter} rows for the GEMM or the calibration kernel under {d}", file=sys.stderr)
            return 1
        factor = CALIB_FLOATS * 4.0 / max(calib)
        res[counter] = {"raw_bytes_per_launch": sum(gemm) / len(gemm), "launches": len(gemm),
                        "calibration_raw_bytes": max(calib), "factor": factor,
                        "bytes_per_launch": sum(gemm) / len(gemm) * factor}
    line = {"kernel": "gemm_kernel", "fetch": res["FETCH_SIZE"], "write": res["WRITE_SIZE"],
            "traffic_bytes_per_launch": res["FETCH_SIZE"]["bytes_per_launch"] + res["WRITE_SIZE"]["bytes_per_launch"]}
    print(json.dumps(line, indent=1))
    return 0


# The stack's GEMM launch kinds, told apart by the kernel's template arguments
# (demangled names) and their order: the q/k/v group runs as a mixed launch,
# gate/up as the fused GLU launch (epilogue kind 2, SwiGLU; persistent
# workgroups when it takes more than one round), O and down as residual
# launches. Down runs as one unsplit round of 128x160 tiles at 2048 tokens,
# the same kernel as O, so there the unsplit residual launches alternate O,
# down, O, ... in the order they were made; where down splits K it is the
# split residual launch and every unsplit one is O.
def gemm_kind(name: str):
    if "gemm_kernel_mixed" in name:
        return "qkv"
    if "gemm_kernel_tiles<" in name:
        return "gate_up" if ", 2>(" in name else "other"
    if "gemm_kernel<" not in name:
        return None
    if ", -2, true>" in name:
        return "down"
    if ", -2, false>" in name:
        return "residual"
    if ", 2, false>" in name or ", 2, true>" in name:
        return "gate_up"
    return "other"


def gemm_kinds(names) -> list:
    """gemm_kind of each kernel name, in dispatch order, with the unsplit
    residual launches resolved into O and down."""
    kinds = [gemm_kind(n) for n in names]
    split_down = "down" in kinds
    r = 0
    for i, k in enumerate(kinds):
        if k == "residual":
            kinds[i] = "o" if split_down or r % 2 == 0 else "down"
            r += 1
    return kinds


def kind_flops(cfg, m: int) -> dict:
    return {"qkv": 2.0 * m * (cfg.q + 2 * cfg.kv) * cfg.hidden, "o": 2.0 * m * cfg.hidden * cfg.q,
            "gate_up": 4.0 * m * cfg.ffn * cfg.hidden, "down": 2.0 * m * cfg.hidden * cfg.ffn}


def counter_summary(args) -> int:
    """Per GEMM launch kind of one prompt step (bench.py --traffic-probe under
    rocprofv3): average duration (--kernel-trace --stats), TFLOP/s and
    fraction of bf16 peak, MFMA-busy share of the SIMD cycles and the clock
    the kernel ran at (SQ_VALU_MFMA_BUSY_CYCLES, GRBM_GUI_ACTIVE; the latter
    is summed over the 8 XCDs), and HBM bytes (FETCH_SIZE, WRITE_SIZE, scaled
    by the calibration kernel as in --traffic-summary)."""
    import csv
    import glob
    from collections import defaultdict
    load_pkg()
    from ggml_xdna_amd.stack import CONFIGS
    cfg = CONFIGS[args.workload]
    m = args.chunk or cfg.chunk
    mfma_dir, fetch_dir, write_dir, trace_dir = args.counter_summary
    sums = defaultdict(lambda: defaultdict(list))
    calib = defaultdict(list)
    for d in (mfma_dir, fetch_dir, write_dir):
        per = defaultdict(float)
        for r in _counter_rows(d):
            per[(int(r["Dispatch_Id"]), r["Kernel_Name"], r["Counter_Name"])] += float(r["Counter_Value"])
        dispatches = sorted({(di, name) for di, name, _ in per})
        kind_of = dict(zip(dispatches, gemm_kinds([name for _, name in dispatches])))
        for (di, name, counter), v in per.items():
            k = kind_of[(di, name)]
            if k:
                sums[k][counter].append(v)
            elif "scale_kernel" in name:
                calib[counter].append(v)
    durs = defaultdict(list)
    for f in glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True):
        rows = sorted(csv.DictReader(open(f)), key=lambda r: int(r["Start_Timestamp"]))
        for r, k in zip(rows, gemm_kinds([r["Kernel_Name"] for r in rows])):
            if k:
                durs[k].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3)
    if not durs or not sums:
        print("no GEMM rows in the given directories", file=sys.stderr)
        return 1
    fl = kind_flops(cfg, m)
    out = {"workload": cfg.name, "chunk": m, "peak_tflops": BF16_PEAK, "simds": 1024, "kinds": {}}
    total_us, total_flops = 0.0, 0.0
    for k in ("qkv", "o", "gate_up", "down"):
        if k not in durs:
            continue
        us = sum(durs[k]) / len(durs[k])
        c = {n: sum(v) / len(v) for n, v in sums[k].items()}
        xcd_cycles = c.get("GRBM_GUI_ACTIVE", 0.0) / 8.0
        row = {"launches": len(durs[k]), "us": round(us, 2), "tflops": round(fl[k] / (us * 1e-6) / 1e12, 1),
               "frac_of_peak": round(fl[k] / (us * 1e-6) / 1e12 / BF16_PEAK, 4)}
        if xcd_cycles > 0 and "SQ_VALU_MFMA_BUSY_CYCLES" in c:
            row["clock_ghz"] = round(xcd_cycles / (us * 1e3), 3)
            row["mfma_busy_pct"] = round(100.0 * c["SQ_VALU_MFMA_BUSY_CYCLES"] / (xcd_cycles * 1024), 1)
            if "SQ_INSTS_MFMA" in c:
                row["mfma_insts"] = int(c["SQ_INSTS_MFMA"])
        for counter, key in (("FETCH_SIZE", "fetch_bytes"), ("WRITE_SIZE", "write_bytes")):
            if counter in c and calib.get(counter):
                factor = CALIB_FLOATS * 4.0 / (max(calib[counter]) * 1024.0)
                row[key] = int(c[counter] * 1024.0 * factor)
        out["kinds"][k] = row
        n_per_step = len(durs[k])
        total_us += us * n_per_step
        total_flops += fl[k] * n_per_step
    out["all_gemm"] = {"us_per_step": round(total_us, 1), "tflops": round(total_flops / (total_us * 1e-6) / 1e12, 1),
                       "frac_of_peak": round(total_flops / (total_us * 1e-6) / 1e12 / BF16_PEAK, 4)}
    print(json.dumps(out, indent=1))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="qwen3-4b")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-tokens", type=int, default=2048)
    ap.add_argument("--unfused", action="store_true", help="gate and up as two GEMMs plus a SwiGLU kernel")
    ap.add_argument("--chunk", type=int, default=None, help="tokens per chunk (default: the workload's)")
    ap.add_argument("--traffic-probe", action="store_true", help="one step and the calibration kernel, for rocprofv3")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"))
    ap.add_argument("--hbm", action="store_true", help="HBM rates of the converter (every type) and the pack")
    ap.add_argument("--kernel-configs", action="store_true",
                    help="BASELINE configs 1 and 2: one Q8_0 MUL_MAT and the SwiGLU FFN triple, launch by launch")
    ap.add_argument("--operand-activity", action="store_true",
                    help="the same GEMM launches on random, workload and all-zero operands (power sensitivity)")
    ap.add_argument("--activity-summary", nargs=2, metavar=("PMC_DIR", "TRACE_DIR"),
                    help="clock and MFMA busy per case from rocprofv3 runs of --operand-activity")
    ap.add_argument("--sustain", type=float, default=None, metavar="SECONDS",
                    help="one GEMM back to back for SECONDS per operand case, for sampling power beside it")
    ap.add_argument("--sustain-kinds", type=float, default=None, metavar="SECONDS",
                    help="the stack's four GEMM launch kinds back to back for SECONDS each, for sampling power")
    ap.add_argument("--sustain-summary", nargs=2, metavar=("PHASES_LOG", "SMI_LOG"),
                    help="power, clock and power-cap status per --sustain phase from amd-smi samples")
    ap.add_argument("--counter-summary", nargs=4, metavar=("MFMA_DIR", "FETCH_DIR", "WRITE_DIR", "TRACE_DIR"),
                    help="per GEMM launch kind: time, MFMA busy, clock, HBM bytes from rocprofv3 runs of --traffic-probe")
    args = ap.parse_args()
    if args.hbm:
        return hbm_kernels(args)
    if args.kernel_configs:
        return kernel_configs(args)
    if args.operand_activity:
        return operand_activity(args)
    if args.activity_summary:
        return activity_summary(*args.activity_summary)
    if args.sustain is not None:
        return sustain(args)
    if args.sustain_kinds is not None:
        return sustain_kinds(args)
    if args.sustain_summary:
        return sustain_summary(*args.sustain_summary)
    if args.counter_summary:
        return counter_summary(args)
    if args.traffic_summary:
        return traffic_summary(*args.traffic_summary)
    if args.traffic_probe:
        return traffic_probe(args)
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
    stack = Stack(cfg, seed=0, fused=not args.unfused, chunk=args.chunk)
    torch.cuda.synchronize()
    print(f"[bench] {cfg.name}: weights converted in {time.perf_counter() - t_build:.1f} s "
          f"(kernel time {stack.convert_ms:.1f} ms)", file=sys.stderr, flush=True)

    for _ in range(args.warmup):
        stack.run_prompt()
    torch.cuda.synchronize()

    t0 = time.perf_counter()
    for _ in range(args.steps):
        stack.run_prompt()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / args.steps

    flops_step = cfg.flops_per_token() * cfg.tokens
    value = flops_step / (ms_step * 1e-3) / 1e12
    # The GEMM kernel's roofline: the same launches back to back, timed with
    # HIP events on the stream they run on (the host ops between them are
    # what the step adds)
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    launches, gemm_flops = 0, 0.0
    for _ in range(args.steps):
        n, f = stack.run_gemms()
        launches += n
        gemm_flops += f
    e1.record(stream)
    e1.synchronize()
    gemm_ms = e0.elapsed_time(e1)
    achieved = gemm_flops / (gemm_ms * 1e-3) / 1e12
    print(f"[bench] {args.steps} steps: {ms_step:.2f} ms/step; the GEMMs alone {gemm_ms / args.steps:.2f} ms/step over "
          f"{launches // args.steps} launches", file=sys.stderr, flush=True)

    # HBM bytes per GEMM launch, from the committed counter runs of this workload
    traffic, traffic_src = None, None
    tf = ROOT / "profiles" / f"gemm_traffic_{cfg.name}.json"
    if tf.exists() and stack.chunk == cfg.chunk and not args.unfused:
        traffic = round(json.loads(tf.read_text())["traffic_bytes_per_launch"])
        traffic_src = str(tf.relative_to(ROOT))
    # MFMA-busy share and clock of the GEMM launches, from the committed counter runs
    counters = None
    cf = ROOT / "profiles" / f"gemm_counters_{cfg.name}.json"
    if cf.exists() and stack.chunk == cfg.chunk and not args.unfused:
        kinds = json.loads(cf.read_text())["kinds"]
        wt = sum(k["us"] * k["launches"] for k in kinds.values())
        counters = {"source": str(cf.relative_to(ROOT)),
                    "mfma_busy_pct": round(sum(k["mfma_busy_pct"] * k["us"] * k["launches"] for k in kinds.values()) / wt, 1),
                    "clock_ghz": round(sum(k["clock_ghz"] * k["us"] * k["launches"] for k in kinds.values()) / wt, 3),
                    "per_kind_frac": {n: k["frac_of_peak"] for n, k in kinds.items()}}
    # board power and clock beside the gate/up GEMM sustained (`--sustain`
    # with amd-smi sampling), from the committed run
    power = None
    pf = ROOT / "profiles" / "gemm_board-power.json"
    if pf.exists() and cfg.name == "qwen3-4b":
        phases = {p["phase"]: p for p in json.loads(pf.read_text()) if p["phase"] != "idle"}
        wl, quiet = phases.get("workload data"), phases.get("W mantissas zero")
        if wl and quiet and wl.get("gfx_clock_mhz") and quiet.get("gfx_clock_mhz"):
            power = {"source": str(pf.relative_to(ROOT)), "board_limit_w": BOARD_POWER_LIMIT_W,
                     "socket_power_w": wl["socket_power_W"], "clock_ghz": round(wl["gfx_clock_mhz"] / 1e3, 3),
                     "quiet_operands": {"socket_power_w": quiet["socket_power_W"],
                                        "clock_ghz": round(quiet["gfx_clock_mhz"] / 1e3, 3),
                                        "speedup": round(quiet["TFLOP/s"] / wl["TFLOP/s"], 3)}}
    # the HBM-bound kernels on rotating sets, as `--hbm` measures them
    names = {v[0]: k for k, v in GGUF_BLOCKS.items()}
    convert = [convert_rate(z, names[t]) for t in dict.fromkeys((cfg.ffn_type, cfg.down_type))]
    pack = pack_rates(z) + [norm_rate(z)]
    # each beside the ceiling it is held against: a device copy moving the
    # same bytes, on rotating sets in the same run
    for r in convert + pack:
        c = copy_rate(r["bytes"])
        r["copy_frac"] = c["frac"]
        r["of_copy"] = round(c["us"] / r["us"], 3)
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
                               f"prompt in {stack.chunk}-token chunks, random-init GGUF weights, attention excluded",
                   "tokens": cfg.tokens, "chunk": stack.chunk, "layers": cfg.layers,
                   "gate_up": "two GEMMs + SwiGLU kernel" if args.unfused else
                              "one fused GEMM, SwiGLU and pack in its epilogue",
                   "operands": "bfp16 (8-value blocks, shared exponent, int8 mantissas) expanded to bf16 for "
                               "MFMA, fp32 accumulate and output"},
        "pct_bf16_peak": round(100 * value / BF16_PEAK, 2),
        "tok_per_s": round(cfg.tokens / (ms_step * 1e-3), 1),
        "roofline": {"bound": "mfma", "kernel": "gemm_kernel", "achieved": round(achieved, 2), "peak": BF16_PEAK,
                     "unit": "TFLOP/s", "frac": round(achieved / BF16_PEAK, 4), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "launches": launches, "avg_launch_us": round(gemm_ms * 1e3 / launches, 2),
                     "timed": "the step's GEMM launches back to back between two HIP events",
                     "counters": counters, "power": power},
        "convert": convert,
        "pack": pack,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(cfg, args.cpu_tokens)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

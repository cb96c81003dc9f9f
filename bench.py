#!/usr/bin/env python3
"""Benchmark of the LARQL quantized compute path on one MI355X.

Headline metric: "Q4_K matvec HBM GB/s (% of peak) + 8B-shape decode tokens/sec".

One step = one pass of the Llama-3-8B FFN matvec trio in 148-byte Q4_K
(gate [14336x4096], up [14336x4096], down [4096x14336]), batch 1, f32
activations, weights drawn N(0, 0.02) on the device and quantized by the
library's device port of the reference quantizer.  Each launch uses one of
16 distinct weight copies (16 x 3 x 34 MB) in rotation so the 256 MB
Infinity Cache cannot serve repeats.  Inputs are resident in HBM before the
timed region; the timed region is bracketed by synchronizations and HIP
events recorded on the stream the kernels are launched on.

value        = algorithmic bytes of all launches / timed wall time (GB/s)
roofline     = the same for the dominant kernel (q4k_matvec) vs 8 TB/s
cpu_baseline = the oracle's port of the reference CPU q4k_matvec, one
               thread, timed on a bounded sample on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "encoding-experiment_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "Q4_K matvec HBM GB/s (% of peak) + 8B-shape decode tokens/sec, 1 GPU"
HBM_PEAK_GBS = 8000.0
SHAPES = (("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336))


def q4k_algorithmic_bytes(rows: int, cols: int) -> int:
    """148-byte Q4_K weights + f32 x + f32 out (one launch)."""
    return rows * (cols // 256) * 148 + cols * 4 + rows * 4


def log(msg: str):
    print(msg, file=sys.stderr, flush=True)


def cpu_baseline(raw_u8, x_np, rows, cols, budget_s: float):
    """Oracle port of LC/src/cpu/ops/q4k_matvec.rs, single thread, bounded sample."""
    import oracle

    runs, t0 = 0, time.perf_counter()
    while True:
        oracle.q4k_matvec(raw_u8, x_np, rows, cols)
        runs += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    gbs = q4k_algorithmic_bytes(rows, cols) * runs / el / 1e9
    return {
        "value": round(gbs, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{runs} x Q4_K matvec [{rows}x{cols}] in {el:.1f} s (oracle port of q4k_matvec.rs, 1 thread)",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=16)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()

    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on exactly one GPU; multi-GPU sharding is design-only "
                                   "(the single-GPU kernels are the per-GPU share of a row-sharded layout)", "n_gpus": args.gpus}))
        sys.exit(2)

    import torch

    import larql_hip

    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)          # kernels, events and torch ops all on this stream
    torch.cuda.set_stream(stream)
    be = larql_hip.HipBackend(0, strict=True)
    log(f"[bench] {be.device_info()}")

    gen = torch.Generator(device=dev)
    handles, xs, outs, raws = {}, {}, {}, {}
    for i, (name, rows, cols) in enumerate(SHAPES):
        gen.manual_seed(1000 + i)
        w = torch.randn(rows, cols, device=dev, generator=gen, dtype=torch.float32) * 0.02
        raw = torch.empty(rows * (cols // 256) * 148, dtype=torch.uint8, device=dev)
        be.quantize_weights_dev(larql_hip.Q4_K, w, rows * cols, raw, stream=stream)
        torch.cuda.synchronize()
        del w
        handles[name] = [be.register_weight_device(larql_hip.Q4_K, raw, raw.numel(), rows, cols)
                         for _ in range(args.copies)]
        raws[name] = raw
        gen.manual_seed(2000 + i)
        xs[name] = torch.randn(cols, device=dev, generator=gen, dtype=torch.float32)
        outs[name] = torch.empty(rows, device=dev, dtype=torch.float32)
    torch.cuda.synchronize()
    log(f"[bench] weights ready: {len(SHAPES)} x {args.copies} copies")

    def step(i):
        for name, _, _ in SHAPES:
            be.matvec_dev(handles[name][i % args.copies], xs[name], outs[name], stream=stream)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record(stream)
    for i in range(args.steps):
        step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1)
    ms_per_step = ms / args.steps
    bytes_per_step = sum(q4k_algorithmic_bytes(r, c) for _, r, c in SHAPES)
    gbs = bytes_per_step * args.steps / (ms * 1e-3) / 1e9
    per_launch_us = ms * 1e3 / (args.steps * len(SHAPES))
    log(f"[bench] {args.steps} steps in {ms:.3f} ms: {ms_per_step * 1e3:.2f} us/step, "
        f"{per_launch_us:.2f} us/launch, {gbs:.1f} GB/s")

    cpu = None
    if not args.no_cpu_baseline:
        name, rows, cols = SHAPES[0]
        cpu = cpu_baseline(raws[name].cpu().numpy(), xs[name].cpu().numpy(), rows, cols, args.cpu_seconds)
        log(f"[bench] cpu baseline: {cpu}")

    per_launch_bytes = q4k_algorithmic_bytes(14336, 4096)
    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: W ~ N(0,0.02) quantized to 148-byte Q4_K on device, x ~ N(0,1)",
        "config": {
            "workload": "Q4_K matvec trio at Llama-3-8B FFN shapes: gate/up [14336x4096], down [4096x14336], batch 1",
            "weight_copies": args.copies,
            "launches_per_step": len(SHAPES),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(per_launch_bytes / (per_launch_us * 1e-6) / 1e9, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(per_launch_bytes / (per_launch_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "q4k_matvec_kernel",
            "bytes_per_launch": per_launch_bytes,
            "avg_launch_us": round(per_launch_us, 3),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    be.close()


if __name__ == "__main__":
    main()

#!/usr/bin/env python3
"""Benchmark of the LARQL quantized compute path on one MI355X.

Headline metric: "Q4_K matvec HBM GB/s (% of peak) + 8B-shape decode tokens/sec, 1 GPU".

Matvec part (the JSON `value`).  One step = one pass of the Llama-3-8B FFN matvec trio
in 148-byte Q4_K (gate [14336x4096], up [14336x4096], down [4096x14336]), batch 1, f32
activations, weights drawn N(0, 0.02) on the device and quantized by the library's
device port of the reference quantizer.  Each launch uses one of 16 distinct weight
copies (16 x 3 x 34 MB) in rotation so the 256 MB Infinity Cache cannot serve
repeats.  Inputs are resident in HBM before the timed region; the timed region is
bracketed by synchronizations and HIP events recorded on the stream the kernels are
launched on.

Decode part (`decode`).  The full synthetic Llama-3-8B Q4_K decode step (32 layers,
d 4096, 32/8 heads, hd 128, FFN 14336, Q6_K head over 128256, fp16 KV prefilled with
2048 positions): the cache is truncated to 2048 before every step, so every timed
step runs at pos 2048; tokens/s = 1 / median step time.

value        = algorithmic bytes of all trio launches / timed wall time (GB/s)
roofline     = the gate launch alone: algorithmic bytes / its average launch time,
               vs 8 TB/s; traffic from the committed rocprofv3 PMC summary
cpu_baseline = the oracle's port of the reference CPU q4k_matvec (q4k_matvec.rs),
               rows split over all the host threads given to this process, timed on
               a bounded sample; cpu_baselines = every workload of the path, one
               thread and all-core, with the host's facts (nproc, CPU model).

PMC helpers (used to produce profiles/q4k_matvec_traffic.json):
  bench.py --pmc-pass calib   plain 64 MiB device copies (known bytes) for scaling
  bench.py --pmc-pass gate    gate-shape Q4_K matvec launches
  bench.py --pmc-pass floor   the plain-read floor kernel over the same gate weights
  bench.py --pmc-pass knn     the Q4_0 gate-KNN walk (34 layers [10240x2560], 256 queries)
  bench.py --pmc-pass walk    the Q4_0 walk-FFN kernels over [10240x2560]
  bench.py --pmc-pass prefill [--pmc-tokens M]  the Q4_K GEMM over [10240x2560] at M tokens
  bench.py --pmc-pass prompt [--pmc-tokens M]   M-token prompt passes through 4 layers of the 8B shape
  bench.py --pmc-report CALIB_FETCH CALIB_WRITE GATE_FETCH GATE_WRITE [--pmc-floor FLOOR_FETCH]
"""
from __future__ import annotations

import argparse
import csv
import json
import os
import statistics
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
TRAFFIC_JSON = os.path.join(ROOT, "profiles", "q4k_matvec_traffic.json")
CALIB_BYTES = 64 << 20
# plain-read floor launch shapes (workgroups, threads); (0, 0) = the matvec's own shape
READ_FLOOR_SHAPES = ((0, 0), (1024, 256), (2048, 256), (4096, 256))


def q4k_algorithmic_bytes(rows: int, cols: int) -> int:
    """148-byte Q4_K weights + f32 x + f32 out (one launch)."""
    return rows * (cols // 256) * 148 + cols * 4 + rows * 4


def decode_algorithmic_bytes(cfg: dict, kv_len: int) -> int:
    """Bytes one decode step must move: Q4_K layer weights, the Q6_K head, the KV
    cache read over T = kv_len + 1 positions, the new K/V row, norms, the embedding
    row and the logits."""
    h, i, nq, nkv, hd, L, V = (cfg[k] for k in ("hidden", "inter", "nq", "nkv", "hd", "n_layers", "vocab"))
    qd, kvd = nq * hd, nkv * hd
    per_layer = sum(r * (c // 256) * 148 for r, c in ((qd, h), (kvd, h), (kvd, h), (h, qd), (i, h), (i, h), (h, i)))
    head = V * (h // 256) * 210
    kv_read = L * (kv_len + 1) * kvd * 2 * 2
    kv_write = L * kvd * 2 * 2
    norms = (2 * L + 1) * h * 4
    return L * per_layer + head + kv_read + kv_write + norms + h * 4 + V * 4


def log(msg: str):
    print(msg, file=sys.stderr, flush=True)


def host_facts(threads: int) -> dict:
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)), "cpu_model": model,
            "threads_all_core": threads}


def all_core_threads() -> int:
    """Threads for the all-core CPU legs: the CPUs this process may run on, capped by
    OMP_NUM_THREADS where the host sets it (the CPU share given to one GPU)."""
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(n, int(env))) if env.isdigit() and int(env) > 0 else n


def _host_blocks(rng, fmt: str, rows: int, cols: int):
    """Random weight bytes in a reference layout with finite, normal f16 scales (the
    CPU kernels' time does not depend on the values)."""
    import numpy as np

    def f16(n, lo, hi):
        return rng.uniform(lo, hi, n).astype(np.float16).view(np.uint8).reshape(-1, 2)

    if fmt == "q8_0":
        return rng.integers(-127, 128, rows * cols, dtype=np.int8), rng.uniform(1e-3, 1e-2, rows * cols // 32).astype(np.float32)
    bpb, per = {"q4_k": (148, 256), "q6_k": (210, 256), "q4_0": (18, 32)}[fmt]
    b = rng.integers(0, 256, (rows * cols // per, bpb), dtype=np.uint8)
    if fmt == "q4_k":
        b[:, 0:2], b[:, 2:4] = f16(len(b), 1e-4, 1e-3), f16(len(b), 1e-4, 1e-3)
    elif fmt == "q6_k":
        b[:, 208:210] = f16(len(b), 1e-4, 1e-3)
    else:
        b[:, 0:2] = f16(len(b), 1e-3, 1e-2)
    return b.reshape(-1), None


def _timed(fn, budget_s: float):
    runs, t0 = 0, time.perf_counter()
    while True:
        fn()
        runs += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            return runs, el


def cpu_baselines(budget_s: float) -> dict:
    """Every workload of the path on this host's CPU through the oracle's ports of the
    reference CPU kernels, one thread and all-core (rows, queries or positions split over
    threads; each slice runs the one-thread kernel, so the outputs are the same).  Each
    leg runs for about budget_s on a bounded sample of the workload, scaled to the unit
    the GPU line reports; `sample` says what ran."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np

    import oracle

    T = all_core_threads()
    pool = ThreadPoolExecutor(T)
    rng = np.random.default_rng(7)
    out = {"host": host_facts(T)}

    def split(rows, fn, nt):
        """fn(r0, r1) over nt contiguous row slices (ctypes calls run without the GIL)."""
        if nt == 1:
            fn(0, rows)
            return
        list(pool.map(lambda t: fn(rows * t // nt, rows * (t + 1) // nt), range(nt)))

    def legs(name, unit, per_run, work, sample, per_time=False):
        """per_run: the unit's amount per call of work(nt) (bytes, flops, walks ...);
        per_time: report seconds (or ms) per unit of per_run instead of a rate."""
        d = {"unit": unit, "sample": sample}
        for label, nt in (("one_thread", 1), ("all_core", T)):
            work(nt)  # warm
            runs, el = _timed(lambda: work(nt), budget_s)
            v = el / (per_run * runs) if per_time else per_run * runs / el
            d[label] = {"value": round(v, 4), "threads": nt, "runs": runs, "seconds": round(el, 2)}
        out[name] = d
        log(f"[bench] cpu {name}: {d}")

    GB = 1e9
    # Q4_K [14336 x 4096] (q4k_matvec.rs), the headline shape
    N, K = 14336, 4096
    w, _ = _host_blocks(rng, "q4_k", N, K)
    x = rng.standard_normal(K).astype(np.float32)
    rb = K // 256 * 148
    legs("q4k_matvec_14336x4096", "GB/s", q4k_algorithmic_bytes(N, K) / GB,
         lambda nt: split(N, lambda a, b: oracle.q4k_matvec(w[a * rb:b * rb], x, b - a, K), nt),
         "one matvec per run")
    # Q4_0 x Q8 [10240 x 2560], the reference's x86 accumulation order (q4_dot.c)
    N, K = 10240, 2560
    w, _ = _host_blocks(rng, "q4_0", N, K)
    xq, xs = oracle.quantize_to_q8(rng.standard_normal(K).astype(np.float32))
    rb = K // 32 * 18
    legs("q4_0_matvec_10240x2560", "GB/s", (N * rb + K + K // 32 * 4 + N * 4) / GB,
         lambda nt: split(N, lambda a, b: oracle.q4_0_matvec_x86(w[a * rb:b * rb], xq, xs, b - a, K), nt),
         "one matvec per run, x86 block order")
    # Q4_0 vecmat [10240 x 2560] (q4_vecmat.rs): out[hidden] accumulates over all rows, so
    # it runs on one thread only
    act = rng.standard_normal(N).astype(np.float32)
    runs, el = _timed(lambda: oracle.q4_0_vecmat(act, w, N, K), budget_s)
    out["q4_0_vecmat_10240x2560"] = {"unit": "GB/s", "sample": "one vecmat per run; one thread (a single "
                                     "accumulation over all rows)",
                                     "one_thread": {"value": round((N * rb + N * 4 + K * 4) * runs / el / GB, 4),
                                                    "threads": 1, "runs": runs, "seconds": round(el, 2)}}
    log(f"[bench] cpu q4_0_vecmat: {out['q4_0_vecmat_10240x2560']}")
    # Q8_0 x Q8 [14336 x 4096], M = 1, 4, 8 (q8_matvec.rs): M matvecs per launch
    N, K = 14336, 4096
    wq, ws = _host_blocks(rng, "q8_0", N, K)
    for m in (1, 4, 8):
        xs8 = [oracle.quantize_to_q8(rng.standard_normal(K).astype(np.float32)) for _ in range(m)]

        def q8run(nt, xs8=xs8):
            def f(a, b):
                for xq_, xs_ in xs8:
                    oracle.q8_matvec(wq[a * K:b * K], ws[a * (K // 32):b * (K // 32)], xq_, xs_, b - a, K)
            split(N, f, nt)

        legs(f"q8_0_matvec_14336x4096_m{m}", "GB/s",
             (N * K + N * K // 32 * 4 + m * (K + K // 32 * 4) + m * N * 4) / GB, q8run,
             f"{m} row(s) per run, bytes counted as the GPU line counts them")
    del wq, ws
    # Q6_K [14336 x 4096] (q6k_matvec.rs)
    w, _ = _host_blocks(rng, "q6_k", N, K)
    rb = K // 256 * 210
    legs("q6k_matvec_14336x4096", "GB/s", (N * rb + K * 4 + N * 4) / GB,
         lambda nt: split(N, lambda a, b: oracle.q6k_matvec(w[a * rb:b * rb], x, b - a, K), nt),
         "one matvec per run")
    # gate-KNN walk: 34 layers [10240 x 2560] x 256 queries, top-32 by |score|
    # (gate_knn.rs); sample: one layer, 8 queries per run, scaled to the whole walk
    L, F, K, Q, k, q_s = 34, 10240, 2560, 256, 32, 8
    g = (rng.standard_normal(F * K) * 0.02).astype(np.float32)
    qs = rng.standard_normal((q_s, K)).astype(np.float32)

    def knn(nt):
        def f(a, b):
            for i in range(a, b):
                oracle.topk_abs(oracle.gate_scores_f32(g, qs[i], F, K), k)
        split(q_s, f, nt)

    legs("gate_knn_f32_34x10240x2560_q256_top32", "s/walk", q_s / (L * Q), knn,
         "1 layer x 8 queries per run (f32 scores + top-32), scaled to 34 layers x 256 queries",
         per_time=True)
    del g
    # prefill GEMM 512 x [10240 x 2560] Q4_K: the reference CPU runs one q4k matvec per
    # position; sample 4 positions per run
    N, K, M, m_s = 10240, 2560, 512, 4
    w, _ = _host_blocks(rng, "q4_k", N, K)
    xs4 = rng.standard_normal((m_s, K)).astype(np.float32)
    rb = K // 256 * 148
    legs("prefill_q4k_gemm_512x10240x2560", "GFLOP/s", 2.0 * m_s * N * K / 1e9,
         lambda nt: split(N, lambda a, b: [oracle.q4k_matvec(w[a * rb:b * rb], xs4[i], b - a, K)
                                           for i in range(m_s)], nt),
         "4 positions per run (one Q4_K matvec each), flops 2 M N K")
    del w
    # 8B-shape decode step at pos 2048: one Q4_K layer per run (the oracle's decode layer,
    # projections row-split over the threads) + the Q6_K head [128256 x 4096] timed on a
    # 16384-row sample; tokens/s = 1 / (32 x layer + head)
    from larql_hip.synth import LLAMA3_8B
    c = LLAMA3_8B
    h, inter, nq, nkv, hd = c["hidden"], c["inter"], c["nq"], c["nkv"], c["hd"]
    qd, kvd, pos = nq * hd, nkv * hd, 2048
    layer = {}
    for name, (r, cc) in dict(wq=(qd, h), wk=(kvd, h), wv=(kvd, h), wo=(h, qd), gate=(inter, h),
                              up=(inter, h), down=(h, inter)).items():
        layer[name] = _host_blocks(rng, "q4_k", r, cc)[0]
    layer["input_norm"] = np.ones(h, np.float32)
    layer["post_attn_norm"] = np.ones(h, np.float32)
    layer["k_cache"] = (rng.standard_normal((pos + 1) * kvd) * 0.5).astype(np.float16).view(np.uint16)
    layer["v_cache"] = (rng.standard_normal((pos + 1) * kvd) * 0.5).astype(np.float16).view(np.uint16)
    hx = rng.standard_normal(h).astype(np.float32)
    hr = 16384
    head, _ = _host_blocks(rng, "q6_k", hr, h)
    d = {"unit": "tokens/s", "sample": f"1 layer at pos {pos} per run x {c['n_layers']} + Q6_K head "
                                       f"{hr}-row sample x {c['vocab'] / hr:.2f}"}
    for label, nt in (("one_thread", 1), ("all_core", T)):
        oracle.decode_layer(layer, hx, pos, h, inter, nq, nkv, hd, 500000.0, threads=nt)
        runs, el = _timed(lambda: oracle.decode_layer(layer, hx, pos, h, inter, nq, nkv, hd, 500000.0,
                                                      threads=nt), budget_s)
        hruns, hel = _timed(lambda: oracle.proj_rows_mt("q6_k", head, hx, hr, h, nt), budget_s / 2)
        step = c["n_layers"] * el / runs + (hel / hruns) * c["vocab"] / hr
        d[label] = {"value": round(1.0 / step, 4), "threads": nt, "s_per_token": round(step, 3),
                    "layer_ms": round(el / runs * 1e3, 2), "head_ms": round(hel / hruns * c["vocab"] / hr * 1e3, 2)}
    out["decode_llama3_8b_q4k_pos2048"] = d
    log(f"[bench] cpu decode: {d}")
    pool.shutdown()
    return out


def make_weights(be, torch, stream, copies):
    import larql_hip

    dev = torch.device("cuda:0")
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
                         for _ in range(copies)]
        raws[name] = raw
        gen.manual_seed(2000 + i)
        xs[name] = torch.randn(cols, device=dev, generator=gen, dtype=torch.float32)
        outs[name] = torch.empty(rows, device=dev, dtype=torch.float32)
    torch.cuda.synchronize()
    return handles, xs, outs, raws


def time_launches(torch, stream, fn, n):
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(n):
        fn(i)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1)  # ms


def run_decode(be, torch, stream, steps, warmup):
    from larql_hip.synth import LLAMA3_8B, build_llama

    sm = build_llama(be, torch, **LLAMA3_8B)
    kv_len = sm.kv_len

    def step():
        be.kv_truncate(kv_len)
        sm.model.decode_dev(sm.x, logits=sm.logits, stream=stream)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    times = []
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for e0, e1 in ev:
        e0.record(stream)
        step()
        e1.record(stream)
    torch.cuda.synchronize()
    times = [e0.elapsed_time(e1) for e0, e1 in ev]
    med = statistics.median(times)
    nbytes = decode_algorithmic_bytes(sm.cfg, kv_len)
    prefill = run_prompt_prefill(torch, stream, sm)
    be.kv_truncate(0)
    sm.model.close()
    del sm
    torch.cuda.empty_cache()
    # the Q4_K_M mix (V and down projections in Q6_K): the same prompt through the Q6_K GEMM
    sm = build_llama(be, torch, q6k=("wv", "down"), **LLAMA3_8B)
    prefill_km = run_prompt_prefill(torch, stream, sm, q6k=("wv", "down"))
    prefill_km["config"] = "Q4_K_M mix: wv and down in Q6_K, the rest Q4_K"
    be.kv_truncate(0)
    sm.model.close()
    del sm
    torch.cuda.empty_cache()
    return {
        "prefill": prefill,
        "prefill_q4_k_m": prefill_km,
        "tokens_per_s": round(1000.0 / med, 2),
        "ms_per_step_median": round(med, 4),
        "ms_per_step_min": round(min(times), 4),
        "steps": steps,
        "bytes_per_step": nbytes,
        "achieved_GBs": round(nbytes / (med * 1e-3) / 1e9, 1),
        "config": "Llama-3-8B shape, Q4_K linears, Q6_K head (vocab 128256), fp16 KV at pos 2048, batch 1",
    }


def run_prompt_prefill(torch, stream, sm, seq=512, reps=4, q6k=()):
    """A 512-token prompt through the 8B-shape model (larql_hip_model_prefill_dev: per
    layer, f32-accuracy GEMMs over all positions and prompt-mode attention).  The Q4_K
    GEMMs issue two fp16 matrix-core products per f32 product (exact integer weight
    operands against the token operand's fp16 pair), the Q6_K GEMMs three (both operands
    as fp16 pairs); `gemm_mfma_frac` is the fp16 MFMA work those imply, over the pass's
    time, against the 2.5 PFLOP/s dense fp16 peak.  q6k: the projections in Q6_K."""
    c = sm.cfg
    gen = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(seq, c["hidden"], generator=gen, device="cuda", dtype=torch.float32)
    out = torch.empty_like(x)
    sm.model.prefill_dev(x, seq, out, stream=stream)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for e0, e1 in ev:
        e0.record(stream)
        sm.model.prefill_dev(x, seq, out, stream=stream)
        e1.record(stream)
    torch.cuda.synchronize()
    ms = statistics.median(e0.elapsed_time(e1) for e0, e1 in ev)
    h, f, q, kv = c["hidden"], c["inter"], c["nq"] * c["hd"], c["nkv"] * c["hd"]
    per_layer = {"wq": h * q, "wk": h * kv, "wv": h * kv, "wo": q * h, "gate": h * f, "up": h * f, "down": f * h}
    gemm_flop = 2.0 * seq * c["n_layers"] * sum(per_layer.values())
    mfma_flop = 2.0 * seq * c["n_layers"] * sum(n * (3 if k in q6k else 2) for k, n in per_layer.items())
    return {
        "tokens": seq,
        "ms_median": round(ms, 3),
        "tokens_per_s": round(seq / (ms * 1e-3), 1),
        "gemm_TFLOPs": round(gemm_flop / (ms * 1e-3) / 1e12, 1),
        "gemm_mfma_frac": round(mfma_flop / (ms * 1e-3) / 2500e12, 3),
    }


EAGER = False  # set by --eager


def _time_us(torch, stream, fn, n, warm=5):
    """Per-call device time (us) of a single-launch entry point: HIP graph replay of n
    calls, or with --eager a timed Python loop."""
    if EAGER:
        for i in range(warm):
            fn(i)
        return time_launches(torch, stream, fn, n) * 1e3 / n
    return _graph_ms(torch, stream, fn, n, warm) * 1e3 / n


def _graph_ms(torch, stream, fn, n, warm=5):
    """Device time of n calls of fn (ms): captured into one HIP graph (every device
    buffer already exists, so the capture holds only kernel launches), replayed once
    untimed and once timed, with HIP events on the launch stream."""
    for i in range(warm):
        fn(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(n):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1)


def _graph_us(torch, stream, fn, n, reps=10, warm=5):
    """Per-call device time of an entry point that launches several kernels: n calls are
    captured into one HIP graph (every device buffer is allocated by the warm-up calls,
    so the capture holds only kernel launches) and replayed `reps` times.  A Python loop
    of such calls measures the interpreter, not the GPU."""
    for i in range(warm):
        fn(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(n):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * n)


def bench_configs(be, torch, stream, copies: int):
    """The other workloads of the path, each at its full single-GPU shape: Q4_0 x Q8
    [10240x2560]; Q4_0 vecmat [10240x2560] and gate/up pair batch (6 positions);
    Q8_0 x Q8 [14336x4096] at M = 1, 4, 8; Q6_K [14336x4096] and
    [4096x14336]; gate-KNN over 34 layers [10240x2560] x 256 queries, top-32, f32 and
    Q4_0; Q4_K prefill GEMM 512 x [10240x2560]."""
    import numpy as np

    import larql_hip

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    out = {}

    def rnd(*shape, seed, std=1.0):
        gen.manual_seed(seed)
        return torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32) * std

    def hbm(name, nbytes, us, extra=None):
        gbs = nbytes / (us * 1e-6) / 1e9
        d = {"us_per_launch": round(us, 3), "bytes_per_launch": nbytes, "GBs": round(gbs, 1),
             "roofline": {"bound": "hbm", "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)}}
        if extra:
            d.update(extra)
        out[name] = d
        log(f"[bench] {name}: {d}")

    def read_floor(name, hs, shapes):
        """The plain read of the same device bytes (no arithmetic) in the kernel's own
        launch shape (first entry) and in fixed shapes: what memory alone allows."""
        fold = torch.empty(max(g for g, _ in shapes), device=dev, dtype=torch.int32)
        fl = {}
        for g, t in shapes:
            fl[f"{g} x {t}"] = round(_time_us(
                torch, stream, lambda i: be.read_floor_dev(hs[i % len(hs)], fold, g, t, stream=stream), 200), 3)
        own = fl[f"{shapes[0][0]} x {shapes[0][1]}"]
        best = min((v, k) for k, v in fl.items())
        out[name].update({"read_floor_us": fl, "over_own_shape_floor": round(out[name]["us_per_launch"] / own, 3),
                          "read_floor_best_us": best[0], "read_floor_best_shape": best[1]})
        log(f"[bench] {name} read floor: {fl}")

    FIXED_FLOOR_SHAPES = ((1024, 256), (2048, 256), (4096, 256))

    # Q4_0 x Q8, [10240 x 2560]
    N, K = 10240, 2560
    w = rnd(N, K, seed=11, std=0.02)
    raw = torch.empty(N * K // 32 * 18, dtype=torch.uint8, device=dev)
    be.quantize_weights_dev(larql_hip.Q4_0, w, N * K, raw, stream=stream)
    torch.cuda.synchronize()
    hs = [be.register_weight_device(larql_hip.Q4_0, raw, raw.numel(), N, K) for _ in range(copies)]
    x = rnd(K, seed=12)
    xq = torch.empty(K, dtype=torch.int8, device=dev)
    xs = torch.empty(K // 32, dtype=torch.float32, device=dev)
    be.quantize_to_q8_dev(x, K, 1, xq, xs, stream=stream)
    y = torch.empty(N, device=dev)
    us = _time_us(torch, stream, lambda i: be.matvec_dev(hs[i % copies], xq, y, x_scales=xs, stream=stream), 200)
    hbm("q4_0_matvec_10240x2560", N * K // 32 * 18 + K + K // 32 * 4 + N * 4, us)
    # the matvec's shape: 16-lane groups, 16 rows per 256-thread workgroup
    read_floor("q4_0_matvec_10240x2560", hs, ((N // 16, 256),) + FIXED_FLOOR_SHAPES)
    for h in hs:
        be.release_weight(h)
    del w, raw

    # Q4_0 walk FFN at [10240 x 2560]: vecmat (down, act [10240] -> out [2560]) and the
    # gate/up pair batch over 6 positions (the reference's profile shape)
    N, K = 10240, 2560
    hs = []
    for c in range(copies):
        w = rnd(N, K, seed=60 + c % 2, std=0.02)
        raw = torch.empty(N * K // 32 * 18, dtype=torch.uint8, device=dev)
        be.quantize_weights_dev(larql_hip.Q4_0, w, N * K, raw, stream=stream)
        torch.cuda.synchronize()
        hs.append(be.register_weight_device(larql_hip.Q4_0, raw, raw.numel(), N, K))
        del w, raw
    act = rnd(N, seed=62)
    y = torch.empty(K, device=dev)
    us = _graph_us(torch, stream, lambda i: be.vecmat_dev(hs[i % copies], act, y, stream=stream), 64)
    hbm("q4_0_vecmat_10240x2560", N * K // 32 * 18 + N * 4 + K * 4, us,
        {"launches": 2, "timing": "HIP graph replay of 64 calls",
         "note": "reference published: CPU 1.35 ms, Metal 1.84 ms on M3 Max (LC/PERFORMANCE.md:60)"})
    seq = 6
    xs6 = rnd(seq, K, seed=63)
    g6 = torch.empty(seq * N, device=dev)
    u6 = torch.empty(seq * N, device=dev)
    us = _graph_us(torch, stream,
                   lambda i: be.pair_batch_dev(hs[i % copies], hs[(i + 1) % copies], xs6, seq, g6, u6, stream=stream), 64)
    hbm("q4_0_pair_batch_6x10240x2560", 2 * (N * K // 32 * 18) + seq * K * 4 + 2 * seq * N * 4, us,
        {"launches": 2, "timing": "HIP graph replay of 64 calls",
         "note": "quantize 6 rows, then the gate and up Q4_0 matvecs over all 6 rows in one launch"})
    for h in hs:
        be.release_weight(h)

    # Q8_0 x Q8, [14336 x 4096], M in {1, 4, 8}
    N, K = 14336, 4096
    w = rnd(N, K, seed=21, std=0.02)
    wq = torch.empty(N * K, dtype=torch.int8, device=dev)
    wsc = torch.empty(N * K // 32, dtype=torch.float32, device=dev)
    be.quantize_weights_dev(larql_hip.Q8_0, w, N * K, wq, q8_scales=wsc, stream=stream)
    torch.cuda.synchronize()
    hs = [be.register_weight_device(larql_hip.Q8_0, wq, wq.numel(), N, K, dev_q8_scales=wsc)
          for _ in range(copies // 2)]
    for m in (1, 4, 8):
        x = rnd(m, K, seed=22)
        xq = torch.empty(m * K, dtype=torch.int8, device=dev)
        xs = torch.empty(m * K // 32, dtype=torch.float32, device=dev)
        be.quantize_to_q8_dev(x, K, m, xq, xs, stream=stream)
        y = torch.empty(m * N, device=dev)
        us = _time_us(torch, stream, lambda i: be.matvec_dev(hs[i % len(hs)], xq, y, m=m, x_scales=xs, stream=stream),
                      200)
        hbm(f"q8_0_matvec_14336x4096_m{m}", N * K + N * K // 32 * 4 + m * (K + K // 32 * 4) + m * N * 4, us)
        if m == 1:  # the matvec's shape at M = 1: 4-lane groups, 32 rows per 128-thread workgroup
            read_floor("q8_0_matvec_14336x4096_m1", hs, ((N // 32, 128),) + FIXED_FLOOR_SHAPES)
    for h in hs:
        be.release_weight(h)
    del w, wq, wsc

    # Q6_K [14336 x 4096] and [4096 x 14336]
    for (N, K), seed in (((14336, 4096), 31), ((4096, 14336), 32)):
        w = rnd(N, K, seed=seed, std=0.02)
        raw = torch.empty(N * K // 256 * 210, dtype=torch.uint8, device=dev)
        be.quantize_weights_dev(larql_hip.Q6_K, w, N * K, raw, stream=stream)
        torch.cuda.synchronize()
        hs = [be.register_weight_device(larql_hip.Q6_K, raw, raw.numel(), N, K) for _ in range(copies)]
        x = rnd(K, seed=seed + 100)
        y = torch.empty(N, device=dev)
        us = _time_us(torch, stream, lambda i: be.matvec_dev(hs[i % copies], x, y, stream=stream), 200)
        hbm(f"q6k_matvec_{N}x{K}", N * K // 256 * 210 + K * 4 + N * 4, us)
        # the matvec's shapes: two 16-row tiles per 512-thread workgroup at [14336 x 4096],
        # one per 896-thread workgroup at [4096 x 14336]
        own = (N // 32, 512) if N == 14336 else (N // 16, 896)
        read_floor(f"q6k_matvec_{N}x{K}", hs, (own,) + FIXED_FLOOR_SHAPES)
        for h in hs:
            be.release_weight(h)
        del w, raw

    # Q4_K at sizes that amortise the launch ramp and at the decode step's fused gate|up:
    # the Llama-3 vocabulary [128256 x 4096] (295 MB; 2 copies rotate past the 256 MB
    # Infinity Cache) and [28672 x 4096] (68 MB, 16 copies), each beside its read floor
    for (N, K), seed, ncopy, fixed in (((128256, 4096), 41, 2, ((2048, 256), (4096, 256), (8192, 256), (16384, 256))),
                                       ((28672, 4096), 42, copies, FIXED_FLOOR_SHAPES + ((8192, 256),))):
        w = rnd(N, K, seed=seed, std=0.02)
        raw = torch.empty(N * K // 256 * 148, dtype=torch.uint8, device=dev)
        be.quantize_weights_dev(larql_hip.Q4_K, w, N * K, raw, stream=stream)
        torch.cuda.synchronize()
        del w
        hs = [be.register_weight_device(larql_hip.Q4_K, raw, raw.numel(), N, K) for _ in range(ncopy)]
        del raw
        x = rnd(K, seed=seed + 100)
        y = torch.empty(N, device=dev)
        n = 40 if N > 100000 else 200
        us = _time_us(torch, stream, lambda i: be.matvec_dev(hs[i % ncopy], x, y, stream=stream), n)
        sh = be.q4k_launch_shape(hs[0])
        hbm(f"q4k_matvec_{N}x{K}", q4k_algorithmic_bytes(N, K), us,
            {"launch": sh, "weight_copies": ncopy})
        read_floor(f"q4k_matvec_{N}x{K}", hs, ((sh["workgroups"], sh["threads"]),) + fixed)
        out[f"q4k_matvec_{N}x{K}"]["over_best_floor"] = round(us / out[f"q4k_matvec_{N}x{K}"]["read_floor_best_us"], 3)
        for h in hs:
            be.release_weight(h)
        torch.cuda.empty_cache()

    # lm-head KNN, Q4 path (lm_head_knn_backend, LV/src/index/walk.rs:549-583): Q4_0
    # [128256 x 4096], one query, top-5 by signed score (quantize_to_q8 + Q4_0 matvec +
    # top-k); 2 copies of 295 MB rotate past the Infinity Cache
    N, K, k5 = 128256, 4096, 5
    w = rnd(N, K, seed=71, std=0.02)
    raw = torch.empty(N * K // 32 * 18, dtype=torch.uint8, device=dev)
    be.quantize_weights_dev(larql_hip.Q4_0, w, N * K, raw, stream=stream)
    torch.cuda.synchronize()
    del w
    hs = [be.register_weight_device(larql_hip.Q4_0, raw, raw.numel(), N, K) for _ in range(2)]
    del raw
    qv = rnd(K, seed=72)
    ki = torch.empty(k5, device=dev, dtype=torch.int32)
    kv_ = torch.empty(k5, device=dev)
    us = _graph_us(torch, stream, lambda i: be.lm_head_knn_dev(hs[i % 2], qv, 1, k5, ki, kv_, stream=stream), 40)
    hbm("lm_head_knn_q4_0_128256x4096_top5", N * K // 32 * 18 + K * 4 + N * 4, us,
        {"launches": 3, "timing": "HIP graph replay of 40 calls",
         "note": "reference comment: ~1 ms for its Q4 lm-head path (LV/src/index/walk.rs:551)"})
    for h in hs:
        be.release_weight(h)
    torch.cuda.empty_cache()

    # multi_layer_q4_ffn (backend.rs:86-96), the trait call with host buffers: 8 layers of
    # Q4_0 gate/up [10240 x 2560] and down [2560 x 10240], chained; weights uploaded once
    # (cached by host pointer), then each call uploads x and downloads the output
    nl, F, K = 8, 10240, 2560
    host_layers = []
    for l in range(nl):
        t3 = []
        for j, (r, cc) in enumerate(((F, K), (F, K), (K, F))):
            w = rnd(r, cc, seed=800 + 3 * l + j, std=0.05)
            raw = torch.empty(r * cc // 32 * 18, dtype=torch.uint8, device=dev)
            be.quantize_weights_dev(larql_hip.Q4_0, w, r * cc, raw, stream=stream)
            torch.cuda.synchronize()
            t3.append(raw.cpu().numpy())
            del w, raw
        host_layers.append(tuple(t3))
    xh = rnd(K, seed=830).cpu().numpy()
    for _ in range(3):
        assert be.multi_layer_q4_ffn(host_layers, xh, F, K) is not None
    ts = []
    for _ in range(50):
        t0 = time.perf_counter()
        be.multi_layer_q4_ffn(host_layers, xh, F, K)
        ts.append(time.perf_counter() - t0)
    us = statistics.median(ts) * 1e6
    hbm("multi_layer_q4_ffn_8x10240x2560", nl * 3 * (F * K // 32 * 18) + 2 * K * 4, us,
        {"timing": "host wall clock per trait call (median of 50), including the x upload and output download",
         "launches_per_call": 4 * nl})
    del host_layers
    be.synchronize()

    # full_pipeline_q4 (backend.rs:71-84), the trait call with host buffers: 2 layers of the
    # Llama-3-8B shape in Q4_K, 16 positions with causal attention among them
    from larql_hip.synth import LLAMA3_8B
    c8 = LLAMA3_8B
    h8, i8, nq8, nkv8, hd8, seq8 = c8["hidden"], c8["inter"], c8["nq"], c8["nkv"], c8["hd"], 16
    qd8, kvd8 = nq8 * hd8, nkv8 * hd8
    ones8 = np.ones(h8, np.float32)
    keep, layers8 = [], []
    for l in range(2):
        arrs = []
        for j, (r, cc) in enumerate(((qd8, h8), (kvd8, h8), (kvd8, h8), (h8, qd8), (i8, h8), (i8, h8), (h8, i8))):
            w = rnd(r, cc, seed=850 + 8 * l + j, std=0.02)
            raw = torch.empty(r * cc // 256 * 148, dtype=torch.uint8, device=dev)
            be.quantize_weights_dev(larql_hip.Q4_K, w, r * cc, raw, stream=stream)
            torch.cuda.synchronize()
            arrs.append(raw.cpu().numpy())
            del w, raw
        keep.append(arrs)
        layers8.append(larql_hip.make_layer(*arrs, ones8, ones8, head_dim=hd8, num_q_heads=nq8, num_kv_heads=nkv8,
                                            rope_base=c8["rope"]))
    x8 = rnd(seq8, h8, seed=870).cpu().numpy()
    for _ in range(2):
        assert be.full_pipeline_q4(layers8, x8, h8, i8, qd8, kvd8, seq8, nq8, nkv8, hd8, c8["rope"]) is not None
    ts = []
    for _ in range(20):
        t0 = time.perf_counter()
        be.full_pipeline_q4(layers8, x8, h8, i8, qd8, kvd8, seq8, nq8, nkv8, hd8, c8["rope"])
        ts.append(time.perf_counter() - t0)
    ms = statistics.median(ts) * 1e3
    wbytes = sum(a.nbytes for arrs in keep for a in arrs)
    out["full_pipeline_q4_2x_llama3_8b_16pos"] = {
        "ms_per_call": round(ms, 3), "tokens_per_s": round(seq8 / (ms * 1e-3), 1),
        "weight_bytes": wbytes, "weight_GBs": round(wbytes / (ms * 1e-3) / 1e9, 1),
        "timing": "host wall clock per trait call (median of 20), including the activation upload and download",
        "note": "positions 0..15 through 2 Llama-3-8B-shape Q4_K layers, causal attention among them, the decode "
                "cache untouched"}
    log(f"[bench] full_pipeline_q4: {out['full_pipeline_q4_2x_llama3_8b_16pos']}")
    del keep, layers8
    torch.cuda.empty_cache()

    # gate-KNN: 34 layers [10240 x 2560] x 256 queries, top-32
    L, F, K, Q, k = 34, 10240, 2560, 256, 32
    hf, hq = [], []
    for l in range(L):
        g = rnd(F, K, seed=9000 + l, std=0.02)
        hf.append(be.register_weight_device(larql_hip.F32, g, g.numel() * 4, F, K))
        raw = torch.empty(F * K // 32 * 18, dtype=torch.uint8, device=dev)
        be.quantize_weights_dev(larql_hip.Q4_0, g, F * K, raw, stream=stream)
        torch.cuda.synchronize()
        hq.append(be.register_weight_device(larql_hip.Q4_0, raw, raw.numel(), F, K))
        del g, raw
    q = rnd(Q, K, seed=4)
    di = torch.empty(L * Q * k, device=dev, dtype=torch.int32)
    dv = torch.empty(L * Q * k, device=dev)
    flops = 2.0 * L * F * K * Q
    for name, hs, peak, unit in (("f32", hf, 157.3, "TFLOP/s"), ("q4_0", hq, 5000.0, "TOP/s")):
        us = _time_us(torch, stream, lambda i: be.gate_knn_dev(hs, q, Q, k, di, dv, stream=stream), 10, warm=2)
        t = flops / (us * 1e-6) / 1e12
        bound = "valu-fp32" if name == "f32" else "mfma-int8"
        out[f"gate_knn_{name}_34x10240x2560_q256_top32"] = {
            "ms_per_walk": round(us / 1e3, 3), "ops": flops, "achieved": round(t, 1), "unit": unit,
            "roofline": {"bound": bound, "peak": peak, "unit": unit, "frac": round(t / peak, 4)},
            "note": "f32 scores are canonical fma chains (bit-exact, no MFMA) on v_fmac_f32, against the "
                    "published 157.3 TFLOP/s fp32 peak; Q4_0 int32 block dots on v_mfma_i32_16x16x64_i8 vs "
                    "the int8 MFMA peak; walk includes top-32 selection"}
        log(f"[bench] gate_knn {name}: {out[f'gate_knn_{name}_34x10240x2560_q256_top32']}")
    for h in hf + hq:
        be.release_weight(h)

    # prefill: 512 tokens through Q4_K [10240 x 2560] on MFMA
    N, K, M = 10240, 2560, 512
    w = rnd(N, K, seed=51, std=0.02)
    raw = torch.empty(N * K // 256 * 148, dtype=torch.uint8, device=dev)
    be.quantize_weights_dev(larql_hip.Q4_K, w, N * K, raw, stream=stream)
    torch.cuda.synchronize()
    hs = [be.register_weight_device(larql_hip.Q4_K, raw, raw.numel(), N, K) for _ in range(copies)]
    x = rnd(M, K, seed=52)
    y = torch.empty(M * N, device=dev)
    us = _time_us(torch, stream, lambda i: be.matvec_dev(hs[i % copies], x, y, m=M, stream=stream), 100)
    fl = 2.0 * M * N * K
    t = fl / (us * 1e-6) / 1e12
    out["prefill_q4k_gemm_512x10240x2560"] = {
        "us_per_launch": round(us, 2), "flops": fl, "achieved": round(t, 1), "unit": "TFLOP/s",
        "roofline": {"bound": "mfma", "peak": 2500.0, "unit": "TFLOP/s", "frac": round(t / 2500.0, 4)},
        "bytes": N * K // 256 * 148 + M * K * 4 + M * N * 4}
    log(f"[bench] prefill: {out['prefill_q4k_gemm_512x10240x2560']}")
    for h in hs:
        be.release_weight(h)
    del w, raw
    torch.cuda.empty_cache()
    return out


def pmc_pass(which: str, launches: int, tokens: int = 512):
    """Kernels only, for a rocprofv3 --pmc run (no timing output)."""
    import torch

    import larql_hip

    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)
    torch.cuda.set_stream(stream)
    if which == "calib":
        src = torch.empty(CALIB_BYTES // 4, device=dev, dtype=torch.float32).uniform_()
        dst = torch.empty_like(src)
        for _ in range(launches):
            dst.copy_(src)
        torch.cuda.synchronize()
        return
    be = larql_hip.HipBackend(0, strict=True)
    if which == "knn":  # the Q4_0 gate-KNN walk: 34 layers [10240 x 2560], 256 queries, top-32
        L, F, K, Q, k = 34, 10240, 2560, 256, 32
        gen = torch.Generator(device=dev)
        hq = []
        for l in range(L):
            gen.manual_seed(9000 + l)
            g = torch.randn(F, K, generator=gen, device=dev, dtype=torch.float32) * 0.02
            raw = torch.empty(F * K // 32 * 18, dtype=torch.uint8, device=dev)
            be.quantize_weights_dev(larql_hip.Q4_0, g, F * K, raw, stream=stream)
            torch.cuda.synchronize()
            hq.append(be.register_weight_device(larql_hip.Q4_0, raw, raw.numel(), F, K))
            del g, raw
        gen.manual_seed(4)
        q = torch.randn(Q, K, generator=gen, device=dev, dtype=torch.float32)
        di = torch.empty(L * Q * k, device=dev, dtype=torch.int32)
        dv = torch.empty(L * Q * k, device=dev)
        for _ in range(max(1, launches // 10)):
            be.gate_knn_dev(hq, q, Q, k, di, dv, stream=stream)
        torch.cuda.synchronize()
        be.close()
        return
    if which == "prefill":  # the Q4_K GEMM (pack + MFMA) over [10240 x 2560] at `tokens` rows, 8 weight copies
        N, K, copies = 10240, 2560, 8
        gen = torch.Generator(device=dev)
        hs = []
        for i in range(copies):
            gen.manual_seed(50 + i)
            g = torch.randn(N, K, generator=gen, device=dev, dtype=torch.float32) * 0.02
            raw = torch.empty(N * K // 256 * 148, dtype=torch.uint8, device=dev)
            be.quantize_weights_dev(larql_hip.Q4_K, g, N * K, raw, stream=stream)
            torch.cuda.synchronize()
            hs.append(be.register_weight_device(larql_hip.Q4_K, raw, raw.numel(), N, K))
            del g, raw
        x = torch.randn(tokens, K, generator=gen, device=dev)
        y = torch.empty(tokens * N, device=dev)
        for i in range(launches):
            be.matvec_dev(hs[i % copies], x, y, m=tokens, stream=stream)
        torch.cuda.synchronize()
        be.close()
        return
    if which == "prompt":  # `launches` 512-token prompt passes through 4 layers of the 8B shape (Q4_K)
        from larql_hip.synth import LLAMA3_8B, build_llama
        sm = build_llama(be, torch, **dict(LLAMA3_8B, n_layers=4))
        gen = torch.Generator(device=dev)
        gen.manual_seed(3)
        x = torch.randn(tokens, sm.cfg["hidden"], generator=gen, device=dev)
        out = torch.empty_like(x)
        for _ in range(launches):
            sm.model.prefill_dev(x, tokens, out, stream=stream)
        torch.cuda.synchronize()
        sm.model.close()
        be.close()
        return
    if which == "walk":  # the Q4_0 walk-FFN kernels over [10240 x 2560]: vecmat, 6-position pair batch, matvec
        N, K, copies = 10240, 2560, 8
        gen = torch.Generator(device=dev)
        hs = []
        for i in range(copies):
            gen.manual_seed(90 + i)
            g = torch.randn(N, K, generator=gen, device=dev, dtype=torch.float32) * 0.02
            raw = torch.empty(N * K // 32 * 18, dtype=torch.uint8, device=dev)
            be.quantize_weights_dev(larql_hip.Q4_0, g, N * K, raw, stream=stream)
            torch.cuda.synchronize()
            hs.append(be.register_weight_device(larql_hip.Q4_0, raw, raw.numel(), N, K))
            del g, raw
        act = torch.randn(N, generator=gen, device=dev)
        y = torch.empty(K, device=dev)
        x6 = torch.randn(6, K, generator=gen, device=dev)
        g6 = torch.empty(6 * N, device=dev)
        u6 = torch.empty(6 * N, device=dev)
        xq = torch.empty(K, dtype=torch.int8, device=dev)
        xsc = torch.empty(K // 32, device=dev)
        be.quantize_to_q8_dev(torch.randn(K, generator=gen, device=dev), K, 1, xq, xsc, stream=stream)
        y2 = torch.empty(N, device=dev)
        for i in range(launches):
            be.vecmat_dev(hs[i % copies], act, y, stream=stream)
            be.pair_batch_dev(hs[i % copies], hs[(i + 1) % copies], x6, 6, g6, u6, stream=stream)
            be.matvec_dev(hs[i % copies], xq, y2, x_scales=xsc, stream=stream)
        torch.cuda.synchronize()
        be.close()
        return
    handles, xs, outs, _ = make_weights(be, torch, stream, copies=16)
    fold = torch.empty(14336 // 16 + 4, device=dev, dtype=torch.int32)
    for i in range(launches):
        if which == "floor":
            be.read_floor_dev(handles["gate"][i % 16], fold, stream=stream)
        else:
            be.matvec_dev(handles["gate"][i % 16], xs["gate"], outs["gate"], stream=stream)
    torch.cuda.synchronize()
    be.close()


def _pmc_values(path: str, counter: str, name_part: str):
    vals = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] == counter and name_part in r["Kernel_Name"]:
                vals.append(float(r["Counter_Value"]))
    if not vals:
        raise SystemExit(f"{path}: no {counter} rows for kernels matching {name_part!r}")
    return vals


def pmc_report(calib_fetch, calib_write, gate_fetch, gate_write, floor_fetch=None):
    """Scale the gate launches' FETCH_SIZE / WRITE_SIZE (KiB per dispatch) by what the
    same counters read for a plain copy of CALIB_BYTES, and write the traffic summary."""
    kib = CALIB_BYTES / 1024.0
    cf = statistics.median(_pmc_values(calib_fetch, "FETCH_SIZE", "copy"))
    cw = statistics.median(_pmc_values(calib_write, "WRITE_SIZE", "copy"))
    gf = statistics.median(_pmc_values(gate_fetch, "FETCH_SIZE", "q4k_mfma_kernel"))
    gw = statistics.median(_pmc_values(gate_write, "WRITE_SIZE", "q4k_mfma_kernel"))
    f_fetch, f_write = kib / cf, kib / cw
    traffic = (gf * f_fetch + gw * f_write) * 1024.0
    alg = q4k_algorithmic_bytes(14336, 4096)
    out = {
        "kernel": "q4k_mfma_kernel (Q4_K, gate [14336x4096])",
        "calibration": {"copy_bytes": CALIB_BYTES, "fetch_kib_read": cf, "write_kib_read": cw,
                        "fetch_scale": round(f_fetch, 4), "write_scale": round(f_write, 4)},
        "gate": {"fetch_kib_raw": gf, "write_kib_raw": gw},
        "traffic_bytes_per_launch": int(traffic),
        "algorithmic_bytes_per_launch": alg,
        "traffic_over_algorithmic": round(traffic / alg, 4),
    }
    if floor_fetch:
        ff = statistics.median(_pmc_values(floor_fetch, "FETCH_SIZE", "q4k_read_floor_kernel"))
        out["read_floor"] = {"fetch_kib_raw": ff, "fetch_bytes": int(ff * f_fetch * 1024.0),
                             "note": "q4k_read_floor_kernel: the gate weight's device bytes read once, "
                                     "same grid and workgroup size as the matvec"}
    os.makedirs(os.path.dirname(TRAFFIC_JSON), exist_ok=True)
    with open(TRAFFIC_JSON, "w") as f:
        json.dump(out, f, indent=2)
    print(json.dumps(out, indent=2))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=16)
    ap.add_argument("--decode-steps", type=int, default=30)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the non-headline workloads")
    ap.add_argument("--cpu-seconds", type=float, default=1.5, help="per CPU-baseline leg (14 legs)")
    ap.add_argument("--eager", action="store_true", help="time Python-loop launches instead of a HIP graph replay")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--pmc-pass", choices=("calib", "gate", "floor", "knn", "walk", "prefill", "prompt"))
    ap.add_argument("--pmc-tokens", type=int, default=512, help="tokens of the prefill PMC pass")
    ap.add_argument("--pmc-launches", type=int, default=50)
    ap.add_argument("--pmc-report", nargs=4, metavar=("CALIB_FETCH", "CALIB_WRITE", "GATE_FETCH", "GATE_WRITE"))
    ap.add_argument("--pmc-floor", metavar="FLOOR_FETCH", help="with --pmc-report: FETCH_SIZE of the read-floor pass")
    args = ap.parse_args()
    global EAGER
    EAGER = args.eager

    if args.pmc_report:
        pmc_report(*args.pmc_report, floor_fetch=args.pmc_floor)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on exactly one GPU; multi-GPU sharding is not built "
                                   "(one GPU's share is the full single-GPU shape)", "n_gpus": args.gpus}))
        sys.exit(2)
    if args.pmc_pass:
        pmc_pass(args.pmc_pass, args.pmc_launches, args.pmc_tokens)
        return

    import torch

    import larql_hip

    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)          # kernels, events and torch ops all on this stream
    torch.cuda.set_stream(stream)
    be = larql_hip.HipBackend(0, strict=True)
    log(f"[bench] {be.device_info()}")

    handles, xs, outs, raws = make_weights(be, torch, stream, args.copies)
    log(f"[bench] weights ready: {len(SHAPES)} x {args.copies} copies")

    def step(i):
        for name, _, _ in SHAPES:
            be.matvec_dev(handles[name][i % args.copies], xs[name], outs[name], stream=stream)

    # The launches are captured into one HIP graph and replayed: a Python loop of
    # ctypes calls enqueues slower than these kernels run (~8 us per call), so eager
    # timing would measure the interpreter.  --eager times the Python loop instead.
    timer = (lambda fn, n: time_launches(torch, stream, fn, n)) if args.eager else \
        (lambda fn, n: _graph_ms(torch, stream, fn, n))
    for i in range(args.warmup):
        step(i)
    ms = timer(step, args.steps)
    ms_per_step = ms / args.steps
    bytes_per_step = sum(q4k_algorithmic_bytes(r, c) for _, r, c in SHAPES)
    gbs = bytes_per_step * args.steps / (ms * 1e-3) / 1e9
    log(f"[bench] trio: {args.steps} steps in {ms:.3f} ms: {ms_per_step * 1e3:.2f} us/step, {gbs:.1f} GB/s")

    # each shape alone, back-to-back launches; beside it the plain-read floor: the same
    # device bytes read once in the same launch shape, with no arithmetic
    per_shape = {}
    for name, rows, cols in SHAPES:
        n = args.steps
        ms_s = timer(lambda i: be.matvec_dev(handles[name][i % args.copies], xs[name], outs[name], stream=stream), n)
        us = ms_s * 1e3 / n
        fold = torch.empty(8192, device=dev, dtype=torch.int32)
        floors = {}
        for g, t in READ_FLOOR_SHAPES:
            ms_f = timer(lambda i: be.read_floor_dev(handles[name][i % args.copies], fold, g, t, stream=stream), n)
            floors["matvec shape" if g == 0 else f"{g} x {t}"] = round(ms_f * 1e3 / n, 3)
        fus = floors["matvec shape"]
        best = min((v, k) for k, v in floors.items())
        per_shape[name] = {"us_per_launch": round(us, 3),
                           "GBs": round(q4k_algorithmic_bytes(rows, cols) / (us * 1e-6) / 1e9, 1),
                           "read_floor_us": fus, "over_own_shape_floor": round(us / fus, 3),
                           "read_floor_best_us": best[0], "read_floor_best_shape": best[1],
                           "over_best_floor": round(us / best[0], 3),
                           "launch": be.q4k_launch_shape(handles[name][0])}
    log(f"[bench] per shape: {per_shape}")

    for name in handles:
        for h in handles[name]:
            be.release_weight(h)
    del raws
    torch.cuda.empty_cache()

    configs = None
    if not args.no_configs:
        configs = bench_configs(be, torch, stream, args.copies)

    decode = None
    if not args.no_decode:
        decode = run_decode(be, torch, stream, args.decode_steps, warmup=5)
        log(f"[bench] decode: {decode}")

    cpu, cpu_all = None, None
    if not args.no_cpu_baseline:
        cpu_all = cpu_baselines(args.cpu_seconds)
        q, one = cpu_all["q4k_matvec_14336x4096"]["all_core"], cpu_all["q4k_matvec_14336x4096"]["one_thread"]
        cpu = {"value": q["value"], "unit": "GB/s", "cores": q["threads"], "kind": "port",
               "sample": f"{q['runs']} Q4_K matvecs [14336x4096] in {q['seconds']} s, rows split over "
                         f"{q['threads']} threads (oracle port of q4k_matvec.rs); one thread: {one['value']} GB/s"}
        log(f"[bench] cpu baseline: {cpu}")

    gate_bytes = q4k_algorithmic_bytes(14336, 4096)
    gate_us = per_shape["gate"]["us_per_launch"]
    sh = per_shape["gate"]["launch"]
    gate_kernel = (f"q4k_mfma_kernel<{sh['ur']}, {sh['tiles']}, false, 0, {sh['pre']}, "
                   f"{'true' if sh['xb'] else 'false'}> gate [14336x4096], {sh['workgroups']} x {sh['threads']} "
                   f"threads, {sh['rounds']} round(s)")
    achieved = gate_bytes / (gate_us * 1e-6) / 1e9
    traffic = None
    if os.path.exists(TRAFFIC_JSON):
        with open(TRAFFIC_JSON) as f:
            traffic = json.load(f).get("traffic_bytes_per_launch")
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
        "dtype": "u8 (4-bit codes) x i8 digit planes of f32 x, int32 MFMA",
        "data": "synthetic: W ~ N(0,0.02) quantized to 148-byte Q4_K on device, x ~ N(0,1)",
        "config": {
            "workload": "Q4_K matvec trio at Llama-3-8B FFN shapes: gate/up [14336x4096], down [4096x14336], batch 1",
            "weight_copies": args.copies,
            "launches_per_step": len(SHAPES),
            "timing": "python loop, HIP events" if args.eager else "HIP graph replay of all steps, HIP events",
            "per_shape": per_shape,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": gate_kernel,
            "bytes_per_launch": gate_bytes,
            "avg_launch_us": gate_us,
            "read_floor_best_us": per_shape["gate"]["read_floor_best_us"],
            "read_floor_best_shape": per_shape["gate"]["read_floor_best_shape"],
            "frac_of_read_floor": round(per_shape["gate"]["read_floor_best_us"] / gate_us, 4),
            "read_floor_own_shape_us": per_shape["gate"]["read_floor_us"],
            "frac_of_own_shape_floor": round(per_shape["gate"]["read_floor_us"] / gate_us, 4),
        },
        "cpu_baseline": cpu,
        "cpu_baselines": cpu_all,
        "decode": decode,
        "configs": configs,
    }
    print(json.dumps(result), flush=True)
    be.close()


if __name__ == "__main__":
    main()

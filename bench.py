#!/usr/bin/env python3
"""Benchmark of the MI355X block-quantised projection path.

Metric: "Q8_0 decode GEMV GB/s (% HBM peak); prefill GEMM int8
TOPS (% MFMA peak)".

step     One decode token's projections of a Llama-3-8B-shaped model with Q8_0
         weights (BASELINE config 1 shapes, 32 layers + lm_head): per layer
         Q|K|V as one batched GEMV (4096->4096, 4096->1024, 4096->1024), o
         (4096->4096), gate|up as one batched GEMV (4096->14336 x2) and down
         (14336->4096); then lm_head (4096->128256).  7.97 GB of weights, all
         resident in HBM and distinct (no cache reuse between launches), fp32
         N(0,1) activations.  The step's 129 launches are captured once in a
         HIP graph and replayed.
value    whole-step algorithmic bytes (weights + x + y per launch) / step time.
roofline dominant kernel: the Q8_0 GEMV at 4096x14336 (down projection, the
         north-star target shape): 96 back-to-back launches rotating over the
         32 layers' distinct down matrices (2 GB), bracketed by HIP events on
         the launch stream (a spin kernel holds the stream while the host
         queues them), so the average includes the inter-kernel gap.
secondary int8 prefill GEMM at M=2048, gate/up shape
         14336x4096 and down shape 4096x14336, as TOPS vs the int8 MFMA peak.
formats_config3 BASELINE config 3 (Q4_0, Q6_K) plus Q4_K / Q5_K: GEMV GB/s and
         GEMM (M = 512) TOPS at both FFN shapes; and the Q8_0 int8 GEMM at
         M = 32, 128, 512 (the rest of the config 2 sweep).
model_config4 BASELINE config 4 on the device-resident decoder (zq_model.h):
         prefill tok/s for a 512-token prompt and decode tok/s for 128
         greedy tokens of a Llama-3-8B-shaped random-init Q8_0 model.
model_config4_formats the same workload with the projections in Q4_0, Q6_K,
         Q4_K and Q5_K (embedding and output Q8_0): int8 prefill for Q4_0,
         fp32 prefill for the super-block formats.
cpu_baseline the reference's own AVX2 ComputePool path (compiled from the
         reference sources into oracle/_ref) on this host's cores (up to 16
         threads, the box's CPU share), on four layers' projections (0.93 GB);
         falls back to the C oracle if the reference build is absent.
         cpu_baseline_reference_policy repeats it (shorter) with the
         reference's own decode worker count, min(physical cores, 8);
         cpu_host gives nproc, usable CPUs, physical cores and the CPU model.

traffic  HBM bytes per launch of the dominant kernel from two rocprofv3 --pmc
         passes (FETCH_SIZE, WRITE_SIZE) over `bench.py --pmc-workload`, each
         scaled by what the counter reads for a 256 MiB device copy in the
         same run; the committed result is profiles/traffic_gemv_q8_0_4096x14336.json.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
       python bench.py --summarize-trace kernel_trace.csv   (rocprofv3 helper)
       python bench.py --pmc-workload                       (short run for --pmc passes)
       python bench.py --model-only                         (config 4 only, for profiling)
"""
import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA (POP/s x 1000)
FP32_PEAK_TFLOPS = 157.3       # MI355X dense fp32 MFMA
F16_PEAK_TFLOPS = 2500.0       # MI355X dense fp16 / bf16 MFMA

HIDDEN, FFN, KV, VOCAB, LAYERS = 4096, 14336, 1024, 128256, 32


def gemv_bytes(fmt_rb, rows, cols):
    return rows * fmt_rb + 4 * cols + 4 * rows


def summarize_trace(path):
    """Group a rocprofv3 kernel_trace.csv by (kernel, grid, LDS) -> count, avg, total."""
    import csv
    groups = {}
    with open(path) as f:
        for row in csv.DictReader(f):
            name = row.get("Kernel_Name", "?")
            grid = row.get("Grid_Size_X", row.get("Grid_Size", "?"))
            lds = row.get("LDS_Block_Size", row.get("Lds_Size", row.get("LDS_Size", "?")))
            dur = int(row["End_Timestamp"]) - int(row["Start_Timestamp"])
            g = groups.setdefault((name, grid, lds), [])
            g.append(dur)
    print(f"{'count':>6} {'avg_us':>10} {'total_ms':>10}  grid  lds  kernel")
    for (name, grid, lds), d in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        print(f"{len(d):6d} {np.mean(d) / 1e3:10.2f} {sum(d) / 1e6:10.3f}  {grid} {lds}  {name[:110]}")


def summarize_gemm_sweep(path):
    """Attribute a kernel_trace.csv of `--gemm-sweep-workload` to its calls
    (each starts with the activation quantiser) and print per (M, N, K) the
    mean per-call time of every kernel over the last 8 of its 16 calls and the
    GEMM's TOPS (2*M*N*K over the GEMM kernel alone, and over the whole
    call)."""
    import csv
    rows = [r for r in csv.DictReader(open(path))
            if "synth" not in r["Kernel_Name"] and "distribution" not in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    calls, cur = [], None
    for r in rows:
        name = r["Kernel_Name"].replace("void ", "").replace("zq::(anonymous namespace)::", "").split("(")[0]
        if name.startswith("quantize_acts_kernel"):
            cur = []
            calls.append(cur)
        if cur is not None:
            cur.append((name, (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3))
    shapes = [(M, N, K) for N, K in ((FFN, HIDDEN), (HIDDEN, FFN)) for M in (32, 128, 512, 2048)]
    print(f"{'M':>5} {'N x K':>12}  {'gemm kernel':34s} {'gemm_us':>8} {'call_us':>8} {'TOPS_gemm':>9} {'TOPS_call':>9}  other kernels (us)")
    for i, (M, N, K) in enumerate(shapes):
        group = calls[16 * i + 8:16 * i + 16]
        if len(group) < 8:
            break
        names = [n for n, _ in group[0]]
        means = [sum(c[j][1] for c in group) / 8 for j in range(len(names))]
        g = next(j for j, n in enumerate(names) if n.startswith("gemm_"))
        ops = 2.0 * M * N * K
        other = ", ".join(f"{names[j]} {means[j]:.2f}" for j in range(len(names)) if j != g)
        print(f"{M:5d} {N:5d}x{K:<6d}  {names[g]:34s} {means[g]:8.2f} {sum(means):8.2f} "
              f"{ops / means[g] / 1e6:9.1f} {ops / sum(means) / 1e6:9.1f}  {other}")


def pmc_workload():
    """Few launches for rocprofv3 --pmc passes: a 256 MiB device copy (counter
    calibration), the 4096x14336 Q8_0 down GEMV on 4 distinct matrices, the
    int8 GEMM at M=2048 on 3 distinct 14336x4096 matrices, and the Q4_K and Q6_K
    GEMVs 14336x4096 on 3 distinct matrices each."""
    import torch
    from zeninfer_amd import zq
    zq.init()
    dev, Q8 = "cuda:0", zq.Q8_0
    a = torch.ones(64 * 1024 * 1024, device=dev)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()

    def W(rows, cols, seed):
        t = torch.empty(zq.weight_bytes(Q8, rows, cols), dtype=torch.uint8, device=dev)
        zq.synth_weights_dev(Q8, seed, t, rows, cols)
        return t
    ws = [W(HIDDEN, FFN, 10 + i) for i in range(4)]
    x = torch.empty(FFN, device=dev)
    zq.synth_normal_dev(1, x, FFN)
    y = torch.empty(HIDDEN, device=dev)
    torch.cuda.synchronize()
    for w in ws:
        zq.gemv_dev(Q8, w, x, y, HIDDEN, FFN)
    torch.cuda.synchronize()
    del ws
    M, N, K = 2048, FFN, HIDDEN
    wg = [W(N, K, 50 + i) for i in range(3)]
    X = torch.empty(M * K, device=dev)
    zq.synth_normal_dev(2, X, M * K)
    Y = torch.empty(M * N, device=dev)
    wsb = zq.gemm_workspace_bytes(Q8, M, N, K, zq.ACT_INT8)
    wsp = torch.empty(wsb, dtype=torch.uint8, device=dev)
    for w in wg:
        zq.gemm_dev(Q8, w, X, Y, M, N, K, zq.ACT_INT8, wsp, wsb)
    torch.cuda.synchronize()
    del wg
    # Q4_K GEMV 14336x4096 on 3 distinct matrices (the K-quant streaming kernel)
    wk = []
    for i in range(3):
        t = torch.empty(zq.weight_bytes(zq.Q4_K, FFN, HIDDEN), dtype=torch.uint8, device=dev)
        zq.synth_weights_dev(zq.Q4_K, 70 + i, t, FFN, HIDDEN)
        wk.append(t)
    yk = torch.empty(FFN, device=dev)
    torch.cuda.synchronize()
    for t in wk:
        zq.gemv_dev(zq.Q4_K, t, x[:HIDDEN], yk, FFN, HIDDEN)
    torch.cuda.synchronize()
    del wk
    # Q6_K GEMV 14336x4096 on 3 distinct matrices (the Q6_K streaming kernel)
    w6 = []
    for i in range(3):
        t = torch.empty(zq.weight_bytes(zq.Q6_K, FFN, HIDDEN), dtype=torch.uint8, device=dev)
        zq.synth_weights_dev(zq.Q6_K, 80 + i, t, FFN, HIDDEN)
        w6.append(t)
    torch.cuda.synchronize()
    for t in w6:
        zq.gemv_dev(zq.Q6_K, t, x[:HIDDEN], yk, FFN, HIDDEN)
    torch.cuda.synchronize()


def measured_traffic():
    """Traffic per launch of the dominant kernel from the committed profile, or None."""
    path = os.path.join(ROOT, "profiles", "traffic_gemv_q8_0_4096x14336.json")
    try:
        with open(path) as f:
            return int(json.load(f)["per_launch"]["traffic_bytes"])
    except (OSError, KeyError, ValueError):
        return None


def gemm_sweep_workload():
    """Config 2's int8 GEMM sweep for a kernel trace: M = 32, 128, 512, 2048 on
    14336x4096 and 4096x14336 (Q8_0), 16 calls each rotating over 4 distinct
    matrices, fp32 activations already in HBM (each call = quantiser + GEMM
    [+ split-K reduction]).  16 back-to-back calls because the shader clock
    settles lower under sustained MFMA load than in a short burst (the first
    M = 2048 calls run ~15% faster than the later ones); the summary averages
    the last 8, the regime bench.py's event timing measures."""
    import torch
    from zeninfer_amd import zq
    zq.init()
    dev, Q8 = "cuda:0", zq.Q8_0
    for N, K in ((FFN, HIDDEN), (HIDDEN, FFN)):
        ws = []
        for i in range(4):
            t = torch.empty(zq.weight_bytes(Q8, N, K), dtype=torch.uint8, device=dev)
            zq.synth_weights_dev(Q8, 60 + i, t, N, K)
            ws.append(t)
        for M in (32, 128, 512, 2048):
            X = torch.empty(M * K, device=dev)
            zq.synth_normal_dev(3, X, M * K)
            Y = torch.empty(M * N, device=dev)
            wsb = zq.gemm_workspace_bytes(Q8, M, N, K, zq.ACT_INT8)
            wsp = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
            torch.cuda.synchronize()
            for i in range(16):
                zq.gemm_dev(Q8, ws[i % 4], X, Y, M, N, K, zq.ACT_INT8, wsp, wsb)
            torch.cuda.synchronize()
            print(f"[gemm-sweep] M={M} N={N} K={K}: 16 calls", file=sys.stderr, flush=True)
        del ws


def cpu_host():
    """nproc, usable CPUs, physical cores and the CPU model of this host."""
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        import psutil
        physical = psutil.cpu_count(logical=False) or usable
    except Exception:
        physical = usable
    return {"nproc": os.cpu_count(), "usable_cpus": usable, "physical_cores": physical, "model": model}


def cpu_baseline(seconds=10.0, layers=4, workers=None):
    """Reference CPU path (oracle/_ref) on `layers` layers' seven Q8_0
    projections each (~0.93 GB, more than a server CPU's last-level cache).
    `workers` defaults to all usable host CPUs up to 16 (the pool caps at 32,
    compute_pool.cpp:87)."""
    from oracle import oracle as O
    o = O.Oracle()
    kind = "reference"
    try:
        r = O.Reference()
        if not r.has_avx2():
            raise RuntimeError("no AVX2")
    except Exception:
        r, kind = None, "port"
    shapes = [(HIDDEN, HIDDEN), (KV, HIDDEN), (KV, HIDDEN), (HIDDEN, HIDDEN), (FFN, HIDDEN), (FFN, HIDDEN), (HIDDEN, FFN)] * layers
    ws = [o.gen_weights(O.Q8_0, 0xC0 + i, rr, cc) for i, (rr, cc) in enumerate(shapes)]
    xs = {c: o.gen_normal(0xC1 + c, c) for c in (HIDDEN, FFN)}
    nbytes = sum(gemv_bytes(o.row_bytes(O.Q8_0, c), rr, c) for rr, c in shapes)
    if workers is None:
        workers = max(1, min(16, cpu_host()["usable_cpus"], 32))

    def one_pass():
        for w, (rr, cc) in zip(ws, shapes):
            if r is not None:
                r.gemv(O.Q8_0, w, xs[cc], rr, cc, workers)
            else:
                o.gemv_f32(O.Q8_0, w, xs[cc], rr, cc)

    one_pass()
    times, t_end = [], time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 6:
        t0 = time.perf_counter()
        one_pass()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times[1:])
    return {"value": round(nbytes / med / 1e9, 2), "unit": "GB/s", "cores": workers if r is not None else 1,
            "kind": kind,
            "sample": f"{layers} Llama-3-8B layers' Q8_0 decode GEMVs (7 per layer, {nbytes / 1e6:.1f} MB), "
                      f"{len(times)} passes, median of all but the first; "
                      + ("reference quant::gemv (AVX2 + ComputePool) built from its sources"
                         if r is not None else "scalar C oracle")}


def prefill_workers(host):
    """The reference's prefill worker count: max(policy workers,
    min(logical CPUs, 32)) (execution_planner.cpp:16-29), the policy being
    min(logical, physical) CPUs when memory is abundant
    (resource_governor.cpp:52-56); logical CPUs are the usable ones (the
    governor reads the cgroup quota, resource_governor.cpp:40-42)."""
    logical = host["usable_cpus"]
    policy = max(1, min(logical, host["physical_cores"]))
    return max(policy, min(logical, 32))


def cpu_gemm_baseline(host, reps=3):
    """The reference's own quant::gemm / quant::gemv (oracle/_ref: AVX2 +
    ComputePool, its K-blocked fp32 route from tokens*K >= 131072,
    src/quant.cpp:1188-1192) on this host at the prefill worker count:
    BASELINE config 2 (Q8_0, M = 32..2048 on both FFN shapes) and config 3
    (Q4_0 and Q6_K: GEMV and M = 512 GEMM on both shapes).  Median of `reps`
    runs after one warm-up.  The reference CPU GEMM computes with fp32
    activations (there is no int8-activation CPU GEMM)."""
    from oracle import oracle as O
    r = O.Reference()
    if not r.has_avx2():
        raise RuntimeError("no AVX2 on this host")
    o = O.Oracle()
    workers = prefill_workers(host)
    out = {"workers": workers, "policy": "prefill: max(policy, min(logical CPUs, 32)) (execution_planner.cpp:16-29)",
           "kind": "reference", "config2_q8_0_gemm": {}, "config3": {}}

    def med(fn):
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    for (N, K) in ((FFN, HIDDEN), (HIDDEN, FFN)):
        w = o.gen_weights(O.Q8_0, 0x5EED0002, N, K)
        for M in (32, 128, 512, 2048):
            X = o.gen_normal(0x5EED0012 + M, M * K)
            sec = med(lambda: r.gemm(O.Q8_0, w, X, M, N, K, workers))
            out["config2_q8_0_gemm"][f"M={M} N={N} K={K}"] = {"ms": round(sec * 1e3, 2),
                                                               "TOPS": round(2.0 * M * N * K / sec / 1e12, 3)}
        del w
    for fname, fmt in (("Q4_0", O.Q4_0), ("Q6_K", O.Q6_K)):
        res = {}
        for shape, N, K in (("gate/up 14336x4096", FFN, HIDDEN), ("down 4096x14336", HIDDEN, FFN)):
            w = o.gen_weights(fmt, 0x5EED0003, N, K)
            x = o.gen_normal(0x5EED0013, K)
            X = o.gen_normal(0x5EED0014, 512 * K)
            g = med(lambda: r.gemv(fmt, w, x, N, K, workers))
            m = med(lambda: r.gemm(fmt, w, X, 512, N, K, workers))
            res[shape] = {"gemv_ms": round(g * 1e3, 3), "gemv_GB_s": round(gemv_bytes(o.row_bytes(fmt, K), N, K) / g / 1e9, 1),
                          "gemm_M512_ms": round(m * 1e3, 2), "gemm_M512_TOPS": round(2.0 * 512 * N * K / m / 1e12, 3)}
            del w
        out["config3"][fname] = res
    return out


def timed_launches_on(torch, launch, n, skip):
    """Average time per launch of n back-to-back launches (after `skip`
    untimed ones), bracketed by HIP events on the launch stream; a spin
    kernel keeps the stream busy while the host queues them, so host
    launch overhead is not in the interval (inter-kernel gaps are)."""
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(int(3e7))
    for i in range(skip):
        launch(i)
    ev0.record()
    for i in range(skip, skip + n):
        launch(i)
    ev1.record()
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) / n


def format_sweep(torch, zq, dev):
    """BASELINE config 3 (Q4_0, Q6_K) plus the K-quants Q4_K / Q5_K: GEMV
    (batch 1) and GEMM (M = 512) at 4096->14336 and 14336->4096, weights
    generated on the device with the oracle's recipes, rotated over enough
    distinct replicas (>= 320 MB) that no launch reads from the MALL.  The
    GEMM uses each format's default activations: int8 for Q4_0, fp32 for the
    super-block formats (their only reference routes), reported against the
    int8 or the fp32 MFMA peak.  Each GEMV is set beside the plain streaming
    read of the same weight bytes (read_ceiling_us).  Also the Q8_0 GEMM M
    sweep of config 2."""
    out = {}
    X = torch.empty(512 * FFN, device=dev)
    zq.synth_normal_dev(31, X, 512 * FFN)
    xv = torch.empty(FFN, device=dev)
    zq.synth_normal_dev(32, xv, FFN)
    sink = torch.empty(zq.read_probe_sink_bytes(), dtype=torch.uint8, device=dev)
    for fname, fmt in (("Q4_0", zq.Q4_0), ("Q6_K", zq.Q6_K), ("Q4_K", zq.Q4_K), ("Q5_K", zq.Q5_K)):
        res = {}
        for shape, N, K in (("gate/up 14336x4096", FFN, HIDDEN), ("down 4096x14336", HIDDEN, FFN)):
            rb = zq.row_bytes(fmt, K)
            nrep = max(2, -(-320_000_000 // (N * rb)))
            ws = []
            for r in range(nrep):
                t = torch.empty(zq.weight_bytes(fmt, N, K), dtype=torch.uint8, device=dev)
                zq.synth_weights_dev(fmt, 0x5EED0003 + 17 * r, t, N, K)
                ws.append(t)
            y = torch.empty(N, device=dev)
            ms = timed_launches_on(torch, lambda i: zq.gemv_dev(fmt, ws[i % nrep], xv[:K], y, N, K), 4 * nrep, nrep)
            # the same weight bytes read by the plain streaming-read probe, same timing
            rms = timed_launches_on(torch, lambda i: zq.read_probe_dev(ws[i % nrep], N * rb, sink), 4 * nrep, nrep)
            entry = {"gemv_us": round(ms * 1e3, 2), "gemv_GB_s": round(gemv_bytes(rb, N, K) / (ms * 1e-3) / 1e9, 1),
                     "read_ceiling_us": round(rms * 1e3, 2), "frac_of_read_ceiling": round(rms / ms, 4)}
            act = zq.ACT_INT8 if fmt == zq.Q4_0 else zq.ACT_F32
            wsb = zq.gemm_workspace_bytes(fmt, 512, N, K, act)
            wsp = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
            Y = torch.empty(512 * N, device=dev)
            ms = timed_launches_on(torch, lambda i: zq.gemm_dev(fmt, ws[i % nrep], X[: 512 * K], Y, 512, N, K, act,
                                                                wsp, wsb), 2 * nrep, 2)
            tops = 2.0 * 512 * N * K / (ms * 1e-3) / 1e12
            # the MFMA each path runs on: int8; the super-block formats' split-f16
            # products (three f16 MFMA products per multiply-add: both operands
            # split); fp32 otherwise
            if act == zq.ACT_INT8:
                peak, mfma = INT8_PEAK_TOPS, "int8"
            elif fmt in (zq.Q6_K, zq.Q4_K, zq.Q5_K):
                peak, mfma = F16_PEAK_TFLOPS / 3.0, "f16 x3 (split operands)"
            else:
                peak, mfma = FP32_PEAK_TFLOPS, "fp32"
            entry.update({"gemm_M512_ms": round(ms, 4), "gemm_M512_TOPS": round(tops, 1),
                          "gemm_act": "int8" if act == zq.ACT_INT8 else "f32", "gemm_mfma": mfma,
                          "gemm_frac_peak": round(tops / peak, 4)})
            res[shape] = entry
            del ws
            torch.cuda.empty_cache()
        out[fname] = res
    # config 2: Q8_0 GEMM, int8 activations, M sweep
    sweep = {}
    for N, K in ((FFN, HIDDEN), (HIDDEN, FFN)):
        rb = zq.row_bytes(zq.Q8_0, K)
        ws = []
        for r in range(6):
            t = torch.empty(zq.weight_bytes(zq.Q8_0, N, K), dtype=torch.uint8, device=dev)
            zq.synth_weights_dev(zq.Q8_0, 0x5EED0002 + r, t, N, K)
            ws.append(t)
        for M in (32, 128, 512):
            wsb = zq.gemm_workspace_bytes(zq.Q8_0, M, N, K, zq.ACT_INT8)
            wsp = torch.empty(wsb, dtype=torch.uint8, device=dev)
            Y = torch.empty(M * N, device=dev)
            ms = timed_launches_on(torch, lambda i: zq.gemm_dev(zq.Q8_0, ws[i % 6], X[: M * K], Y, M, N, K,
                                                                zq.ACT_INT8, wsp, wsb), 12, 6)
            ops = 2.0 * M * N * K
            wbytes = N * rb + 4 * M * K + 4 * M * N
            sweep[f"M={M} N={N} K={K}"] = {"ms": round(ms, 4), "TOPS": round(ops / (ms * 1e-3) / 1e12, 1),
                                           "GB_s": round(wbytes / (ms * 1e-3) / 1e9, 1)}
        del ws
        torch.cuda.empty_cache()
    out["q8_0_gemm_int8_M_sweep"] = sweep
    return out


def model_config4_formats():
    """Config 4's workload (512-token prompt, 128 greedy tokens, second of two
    runs) with the projections in the other formats; the embedding table and
    the output projection stay Q8_0."""
    import numpy as np
    from zeninfer_amd import zq
    from zeninfer_amd.model import Model, PREFILL_F32, PREFILL_INT8
    prompt = np.random.default_rng(0x5EED0004).integers(0, VOCAB, size=512).tolist()
    out = {}
    for fmt, name in ((zq.Q4_0, "Q4_0"), (zq.Q6_K, "Q6_K"), (zq.Q4_K, "Q4_K"), (zq.Q5_K, "Q5_K")):
        m = Model.synthetic(seed=0x5EED0004, embedding=HIDDEN, layers=LAYERS, heads=32, kv_heads=8, ffn=FFN,
                            vocab=VOCAB, context=8192, max_positions=1024, rope_base=500000.0, rms_epsilon=1e-5,
                            eos_token=0xFFFFFFFF, weight_format=fmt)
        m.set_prefill_mode(PREFILL_INT8 if fmt == zq.Q4_0 else PREFILL_F32)
        for _ in range(2):
            toks, pm, dm = m.generate(prompt, 128)
        mem = m.memory()
        m.close()
        steps = len(toks) - 1
        out[name] = {"prefill": "int8" if fmt == zq.Q4_0 else "f32", "prefill_tok_s": round(512 / (pm * 1e-3), 1),
                     "decode_tok_s": round(steps / (dm * 1e-3), 1), "weights_bytes": mem["weights"],
                     "decode_weight_GB_s": round(mem["weights"] / (dm / steps * 1e-3) / 1e9, 1)}
    return out


def model_config4():
    """BASELINE config 4 through the device-resident decoder (include/zq_model.h):
    a random-init Llama-3-8B-shaped Q8_0 model generated on the device (no
    8.5 GB file), a 512-token random prompt (seeded), then 128 greedily decoded
    tokens (EOS disabled so all 128 are produced).  Two runs; the second is
    reported (the first captures the decode graph)."""
    import numpy as np
    from zeninfer_amd.model import Model, PREFILL_INT8
    m = Model.synthetic(seed=0x5EED0004, embedding=HIDDEN, layers=LAYERS, heads=32, kv_heads=8, ffn=FFN,
                        vocab=VOCAB, context=8192, max_positions=1024, rope_base=500000.0, rms_epsilon=1e-5,
                        eos_token=0xFFFFFFFF)
    m.set_prefill_mode(PREFILL_INT8)
    prompt = np.random.default_rng(0x5EED0004).integers(0, VOCAB, size=512).tolist()
    for _ in range(2):
        toks, pm, dm = m.generate(prompt, 128)
    mem = m.memory()
    m.close()
    steps = len(toks) - 1
    return {"workload": "config 4: Llama-3-8B-shaped dense forward, random-init Q8_0 weights generated on the device, "
                        "512-token random prompt, 128 greedy tokens (int8-activation prefill GEMM, fp32 GEMV decode, "
                        "decode step replayed as one HIP graph)",
            "prefill_ms": round(pm, 2), "prefill_tok_s": round(512 / (pm * 1e-3), 1),
            "decode_ms_per_token": round(dm / steps, 4), "decode_tok_s": round(steps / (dm * 1e-3), 1),
            "tokens": len(toks), "weights_bytes": mem["weights"], "kv_cache_bytes": mem["kv_cache"],
            "decode_weight_GB_s": round(mem["weights"] / (dm / steps * 1e-3) / 1e9, 1)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--summarize-trace")
    ap.add_argument("--summarize-gemm-sweep")
    ap.add_argument("--pmc-workload", action="store_true")
    ap.add_argument("--gemm-sweep-workload", action="store_true",
                    help="only config 2's int8 GEMM sweep, 3 calls per shape (kernel-trace helper)")
    ap.add_argument("--model-only", action="store_true",
                    help="run only the config-4 decoder leg and print its JSON (profiling helper)")
    ap.add_argument("--model-formats-only", action="store_true",
                    help="run only the config-4 decoder leg in Q4_0 / Q6_K / Q4_K / Q5_K and print its JSON")
    args = ap.parse_args()
    if args.summarize_trace:
        summarize_trace(args.summarize_trace)
        return 0
    if args.summarize_gemm_sweep:
        summarize_gemm_sweep(args.summarize_gemm_sweep)
        return 0
    if args.pmc_workload:
        pmc_workload()
        return 0
    if args.gemm_sweep_workload:
        gemm_sweep_workload()
        return 0
    if args.model_only:
        import torch
        from zeninfer_amd import zq
        torch.cuda.set_device(0)
        zq.init()
        print(json.dumps(model_config4()))
        return 0
    if args.model_formats_only:
        import torch
        from zeninfer_amd import zq
        torch.cuda.set_device(0)
        zq.init()
        print(json.dumps(model_config4_formats()))
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU leg (the projections would shard "
              "by weight rows, one process per GPU; that is a design, not code)", file=sys.stderr)
        return 2

    import torch
    from zeninfer_amd import zq
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    st = zq.init()
    if st != 0:
        raise RuntimeError(f"zq_hip_init: {zq.status_string(st)}")
    info = zq.info()
    Q8 = zq.Q8_0
    rbh, rbf = zq.row_bytes(Q8, HIDDEN), zq.row_bytes(Q8, FFN)

    def weights(rows, cols, seed):
        t = torch.empty(zq.weight_bytes(Q8, rows, cols), dtype=torch.uint8, device=dev)
        zq.synth_weights_dev(Q8, seed, t, rows, cols)
        return t

    print(f"[bench] device {info['name']} {info['arch']} CUs={info['compute_units']}", file=sys.stderr, flush=True)
    layers = []
    for l in range(LAYERS):
        s = 1000 * (l + 1)
        layers.append({"q": weights(HIDDEN, HIDDEN, s + 1), "k": weights(KV, HIDDEN, s + 2),
                       "v": weights(KV, HIDDEN, s + 3), "o": weights(HIDDEN, HIDDEN, s + 4),
                       "gate": weights(FFN, HIDDEN, s + 5), "up": weights(FFN, HIDDEN, s + 6),
                       "down": weights(HIDDEN, FFN, s + 7)})
    lm_head = weights(VOCAB, HIDDEN, 7)
    x_h = torch.empty(HIDDEN, device=dev)
    x_f = torch.empty(FFN, device=dev)
    zq.synth_normal_dev(11, x_h, HIDDEN)
    zq.synth_normal_dev(12, x_f, FFN)
    y_q, y_k, y_v, y_o = (torch.empty(n, device=dev) for n in (HIDDEN, KV, KV, HIDDEN))
    y_g, y_u, y_d = (torch.empty(n, device=dev) for n in (FFN, FFN, HIDDEN))
    y_lm = torch.empty(VOCAB, device=dev)
    torch.cuda.synchronize()
    print("[bench] weights generated", file=sys.stderr, flush=True)

    stream = torch.cuda.current_stream()

    def step():
        for L in layers:
            zq.gemv_batch_dev(Q8, x_h, [(L["q"], y_q, HIDDEN), (L["k"], y_k, KV), (L["v"], y_v, KV)], HIDDEN, stream)
            zq.gemv_dev(Q8, L["o"], x_h, y_o, HIDDEN, HIDDEN, stream)
            zq.gemv_batch_dev(Q8, x_h, [(L["gate"], y_g, FFN), (L["up"], y_u, FFN)], HIDDEN, stream)
            zq.gemv_dev(Q8, L["down"], x_f, y_d, HIDDEN, FFN, stream)
        zq.gemv_dev(Q8, lm_head, x_h, y_lm, VOCAB, HIDDEN, stream)

    layer_bytes = (gemv_bytes(rbh, HIDDEN, HIDDEN) * 2 + gemv_bytes(rbh, KV, HIDDEN) * 2
                   + gemv_bytes(rbh, FFN, HIDDEN) * 2 + gemv_bytes(rbf, HIDDEN, FFN))
    # batched launches read x once: subtract the duplicate x reads of the batch members
    layer_bytes -= 4 * HIDDEN * 2 + 4 * HIDDEN * 1
    step_bytes = LAYERS * layer_bytes + gemv_bytes(rbh, VOCAB, HIDDEN)

    # eager reference output, then capture the step as a graph
    step()
    torch.cuda.synchronize()
    eager_lm = y_lm.clone()
    eager_d = y_d.clone()
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(stream)
    with torch.cuda.stream(cap):
        with torch.cuda.graph(graph, stream=cap):
            stream = cap
            step()
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    for _ in range(max(1, args.warmup)):
        graph.replay()
    torch.cuda.synchronize()
    graph_ok = bool(torch.equal(y_lm, eager_lm) and torch.equal(y_d, eager_d))

    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record()
    for _ in range(args.steps):
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    ms_step = ev0.elapsed_time(ev1) / args.steps
    value = step_bytes / (ms_step * 1e-3) / 1e9
    print(f"[bench] step {ms_step:.3f} ms  {value:.1f} GB/s  graph_ok={graph_ok}", file=sys.stderr, flush=True)

    # ---- roofline leg: per-launch timing of the 4096 x 14336 down GEMV ----
    timed_launches = lambda launch, n, skip: timed_launches_on(torch, launch, n, skip)

    down_bytes = gemv_bytes(rbf, HIDDEN, FFN)
    down_ms = timed_launches(lambda i: zq.gemv_dev(Q8, layers[i % LAYERS]["down"], x_f, y_d, HIDDEN, FFN),
                             4 * LAYERS, LAYERS)
    down_gbs = down_bytes / (down_ms * 1e-3) / 1e9
    # the practical ceiling of one launch that reads the same weight bytes: a
    # plain non-temporal streaming read (no compute) of each down matrix,
    # timed the same way (zq_hip_read_probe_dev)
    sink = torch.empty(zq.read_probe_sink_bytes(), dtype=torch.uint8, device=dev)
    wbytes = HIDDEN * rbf
    read_ms = timed_launches(lambda i: zq.read_probe_dev(layers[i % LAYERS]["down"], wbytes, sink), 4 * LAYERS, LAYERS)
    read_gbs = wbytes / (read_ms * 1e-3) / 1e9

    # per-shape GB/s (informational), same method
    per_shape = {}
    for name, key, rows, cols, x in (("q/o 4096x4096", "q", HIDDEN, HIDDEN, x_h), ("k/v 1024x4096", "k", KV, HIDDEN, x_h),
                                     ("gate/up 14336x4096", "gate", FFN, HIDDEN, x_h),
                                     ("down 4096x14336", "down", HIDDEN, FFN, x_f)):
        yb = torch.empty(rows, device=dev)
        ms = timed_launches(lambda i: zq.gemv_dev(Q8, layers[i % LAYERS][key], x, yb, rows, cols), 2 * LAYERS, LAYERS)
        # the same weight bytes read by the plain streaming-read probe, same timing
        wb = rows * zq.row_bytes(Q8, cols)
        rms = timed_launches(lambda i: zq.read_probe_dev(layers[i % LAYERS][key], wb, sink), 2 * LAYERS, LAYERS)
        per_shape[name] = {"us": round(ms * 1e3, 2),
                           "GB/s": round(gemv_bytes(zq.row_bytes(Q8, cols), rows, cols) / (ms * 1e-3) / 1e9, 1),
                           "read_ceiling_us": round(rms * 1e3, 2), "frac_of_read_ceiling": round(rms / ms, 4)}
    ms = timed_launches(lambda i: zq.gemv_dev(Q8, lm_head, x_h, y_lm, VOCAB, HIDDEN), 8, 1)
    rms = timed_launches(lambda i: zq.read_probe_dev(lm_head, VOCAB * rbh, sink), 8, 1)
    per_shape["lm_head 128256x4096"] = {"us": round(ms * 1e3, 2),
                                        "GB/s": round(gemv_bytes(rbh, VOCAB, HIDDEN) / (ms * 1e-3) / 1e9, 1),
                                        "read_ceiling_us": round(rms * 1e3, 2),
                                        "frac_of_read_ceiling": round(rms / ms, 4)}

    # ---- secondary: int8 prefill GEMM at M = 2048 (config 2) ---------------
    M = 2048
    X = torch.empty(M * FFN, device=dev)
    zq.synth_normal_dev(21, X, M * FFN)
    gemm = {}
    for name, key, N, K in (("gate/up 14336x4096", "gate", FFN, HIDDEN), ("down 4096x14336", "down", HIDDEN, FFN)):
        wsb = zq.gemm_workspace_bytes(Q8, M, N, K, zq.ACT_INT8)
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        Y = torch.empty(M * N, device=dev)
        Xk = X[: M * K]
        xq = torch.empty(M * K, dtype=torch.int8, device=dev)
        xs = torch.empty(M * K // 32, device=dev)
        full_ms = timed_launches(lambda i: zq.gemm_dev(Q8, layers[i % 8][key], Xk, Y, M, N, K, zq.ACT_INT8, ws, wsb),
                                 16, 8)
        q_ms = timed_launches(lambda i: zq.quantize_acts_dev(Xk, xq, xs, M, K), 16, 4)
        ops = 2.0 * M * N * K
        k_ms = full_ms - q_ms
        gemm[name] = {"shape": f"M={M} N={N} K={K}", "ms_per_call": round(full_ms, 4), "quantize_ms": round(q_ms, 4),
                      "gemm_ms": round(k_ms, 4),
                      "TOPS_per_call": round(ops / (full_ms * 1e-3) / 1e12, 1),
                      "TOPS_gemm": round(ops / (k_ms * 1e-3) / 1e12, 1),
                      "frac_int8_peak": round(ops / (k_ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4)}

    # ---- the int8 peak from measurement (MFMA rate x CUs x sclk) -----------
    sclk_mhz, cyc_per_mfma, int8_peak_meas = zq.mfma_peak()
    # the GEMM's own arithmetic floor: per 32x32 output tile and 32-element K
    # block (65536 int8 ops) one int8 MFMA (32 cycles), half of a 2-block
    # scale MFMA (32 cycles) and 16 cvt + 16 fma VALU at 2.2 cycles each
    # (measured issue rates; MFMA and VALU do not overlap on one SIMD)
    floor_cycles = 32.0 + 32.0 + 32 * 2.2
    valu_floor_tops = info["compute_units"] * 4 * 65536.0 / floor_cycles * sclk_mhz * 1e6 / 1e12
    for g in gemm.values():
        g["frac_measured_int8_peak"] = round(g["TOPS_per_call"] / int8_peak_meas, 4)
        g["frac_epilogue_floor"] = round(g["TOPS_per_call"] / valu_floor_tops, 4)

    # ---- config 3 formats + config 2 M sweep ----------------------------------
    formats = format_sweep(torch, zq, dev)
    print(f"[bench] formats {json.dumps(formats)}", file=sys.stderr, flush=True)

    # ---- config 4: the device-resident decoder, prefill 512 + 128 greedy tokens
    model4 = model_config4()
    model4_formats = model_config4_formats()
    print(f"[bench] config-4 formats {json.dumps(model4_formats)}", file=sys.stderr, flush=True)

    cpu = cpu_policy = host = cpu_gemm = None
    if not args.no_cpu:
        try:
            cpu = cpu_baseline(seconds=8.0)
            host = cpu_host()
            # the reference's own decode policy: min(physical cores, 8) workers
            # (execution_planner.cpp:22-28), a shorter sample
            pw = max(1, min(host["physical_cores"], host["usable_cpus"], 8))
            pol = cpu_baseline(seconds=4.0, workers=pw)
            cpu_policy = {"value": pol["value"], "unit": pol["unit"], "cores": pol["cores"], "kind": pol["kind"],
                          "policy": "decode: min(physical cores, 8) workers (execution_planner.cpp:22-28)"}
        except Exception as e:  # reported, never fatal to the GPU measurement
            cpu = {"error": str(e)}
        try:
            cpu_gemm = cpu_gemm_baseline(host or cpu_host())
        except Exception as e:
            cpu_gemm = {"error": str(e)}

    out = {
        "metric": "Q8_0 decode GEMV GB/s (% HBM peak); prefill GEMM int8 TOPS (% MFMA peak)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded SplitMix64/Box-Muller Q8_0 weights generated on the device, N(0,1) fp32 activations)",
        "config": {"workload": "config 1: Llama-3-8B-shaped Q8_0 decode projections, batch 1, one token = "
                               "32 layers x (QKV batch, o, gate|up batch, down) + lm_head, HIP-graph replay",
                   "weights_bytes_per_step": int(step_bytes), "launches_per_step": LAYERS * 4 + 1,
                   "frac_hbm_peak_step": round(value / HBM_PEAK_GBS, 4), "graph_matches_eager": graph_ok},
        "roofline": {"bound": "hbm", "achieved": round(down_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(down_gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "kernel": "gemv_mfma_kernel<Q8_0> (int8 MFMA on the exact digit split of x) at 4096x14336, the down projection",
                     "avg_launch_us": round(down_ms * 1e3, 2), "algorithmic_bytes_per_launch": down_bytes,
                     "read_ceiling": {"us": round(read_ms * 1e3, 2), "GB/s": round(read_gbs, 1),
                                      "frac": round(read_gbs / HBM_PEAK_GBS, 4),
                                      "what": "plain streaming read of the same weight bytes, one launch each, "
                                              "same timing (zq_hip_read_probe_dev)"},
                     "frac_of_read_ceiling": round(down_gbs / read_gbs, 4)},
        "per_shape_gemv": per_shape,
        "secondary": {"metric": "prefill GEMM int8 TOPS (% MFMA peak), config 2 at M=2048",
                      "prefill_gemm_int8_M2048": gemm, "int8_peak_tops": INT8_PEAK_TOPS,
                      "int8_peak_measured": {"tops": round(int8_peak_meas, 1), "sclk_mhz": round(sclk_mhz, 1),
                                             "cycles_per_mfma_i32_32x32x32_i8": round(cyc_per_mfma, 2),
                                             "derivation": "CUs x 4 SIMDs x 65536 ops / cycles per MFMA x measured sclk"},
                      "roofline_epilogue_floor": {"tops": round(valu_floor_tops, 1),
                                                  "cycles_per_tile_block": floor_cycles,
                                                  "derivation": "int8 MFMA 32 + half a 2-block scale MFMA 32 + "
                                                                "(16 cvt + 16 fma) x 2.2 cycles per 32x32x32 tile-block"}},
        "formats_config3": formats,
        "model_config4": model4,
        "model_config4_formats": model4_formats,
        "cpu_baseline": cpu,
        "cpu_baseline_reference_policy": cpu_policy,
        "cpu_baseline_gemm_and_config3": cpu_gemm,
        "cpu_host": host,
    }
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())

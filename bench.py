#!/usr/bin/env python3
"""Benchmark of the fp32 GEMM hot path on one MI355X.

Default workload (BASELINE.json metric "fp32 GEMM TFLOP/s @4096^3"): nn::kernels::sgemm's replacement,
C = A B with A, B 4096 x 4096 fp32 from the reference's own seeded uniform[-1, 1] stream (seed 4, A filled
first, then B: apps/bench/runner.cpp:80-86). One step = one 4096^3 product; inputs are resident in HBM
before timing starts. Prints one JSON line on stdout (diagnostics go to stderr).

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

roofline.achieved = 2 M N K / (average kernel duration from HIP events recorded on the launch stream);
roofline.traffic comes from the committed rocprofv3 PMC summary (profiles/sgemm_4096_pmc.md) when present.
cpu_baseline = nn-cpp's NN_NATIVE AVX2 sgemm (oracle/_ref, compiled from the reference's own sources) on the
same inputs, on the host's cores (at most 16 threads), median of a bounded number of runs.
"""
import argparse
import json
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "nn-cpp_amd"))

PEAK_FP32_MFMA_TFLOPS = 157.3   # MI355X dense fp32 matrix peak (AMD spec)
PEAK_HBM_GBPS = 8000.0          # MI355X HBM3E


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def traffic_from_profile(name):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, copy-calibrated)."""
    path = os.path.join(ROOT, "profiles", f"{name}_pmc.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"hbm_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read())
    return float(m.group(1)) if m else None


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def cpu_baseline(a, b, m, n, k, budget_s=12.0, max_runs=30):
    """nn-cpp's own sgemm (oracle/_ref) on the same host buffers, reference method: warm-up, then the median of
    timed runs (apps/bench/runner.cpp:80-96), bounded to about budget_s seconds of CPU work."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    from pyoracle import Reference, reference_available
    if not reference_available():
        log("cpu_baseline: oracle/_ref not built; skipped")
        return None
    ref = Reference()
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    threads = max(1, min(16, avail))
    ref.set_threads(threads)
    c = np.empty((m, n), np.float32)
    ref.sgemm_inplace(0, 0, m, n, k, a, k, b, n, c, n, 0)  # warm-up (pool start, page faults)
    times = []
    t_start = time.perf_counter()
    while len(times) < max_runs and (time.perf_counter() - t_start) < budget_s:
        t0 = time.perf_counter()
        ref.sgemm_inplace(0, 0, m, n, k, a, k, b, n, c, n, 0)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {
        "value": round(2.0 * m * n * k / med / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "reference",
        "sample": (f"nn::kernels::sgemm {m}x{n}x{k} NN (nn-cpp 2.0.0 NN_NATIVE AVX2/FMA build, -O3 -mavx2 -mfma "
                   f"-ffp-contract=off), same seed-4 inputs, {threads} threads on {cpu_model()}, median of "
                   f"{len(times)} runs after 1 warm-up ({sum(times):.1f} s timed)"),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--size", type=int, default=4096)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); --gpus {args.gpus} is not "
              "supported", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import nnh
    from nnh import synth

    m = n = k = args.size
    a, b = synth.uniform_operands(4, [(m, k), (k, n)])
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    dev = torch.device("cuda:0")
    da, db = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
    dc = torch.empty((m, n), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream()

    def step():
        nnh.sgemm(0, 0, m, n, k, da, k, db, n, dc, n, 0, stream=stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kernel_ms = ev0.elapsed_time(ev1) / args.steps
    flops = 2.0 * m * n * k
    value = flops * args.steps / wall / 1e12
    achieved = flops / (kernel_ms * 1e-3) / 1e12
    log(f"sgemm {m}^3: {kernel_ms:.4f} ms/launch (HIP events), {achieved:.2f} TFLOP/s per launch, "
        f"{value:.2f} TFLOP/s wall over {args.steps} steps")

    cpu = None if args.no_cpu_baseline else cpu_baseline(a, b, m, n, k)
    if cpu:
        log(f"cpu baseline: {cpu['value']} TFLOP/s ({cpu['sample']})")
    traffic = traffic_from_profile(f"sgemm_{m}")
    out = {
        "metric": "fp32 GEMM TFLOP/s @4096^3 (nn::kernels::sgemm replacement, bit-exact with nn-cpp)",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: the reference's seeded uniform[-1,1] stream (std::mt19937(4) + "
                "uniform_real_distribution<float>), A then B",
        "config": {"workload": f"sgemm {m}x{n}x{k} NN fp32 (BASELINE config 5)", "m": m, "n": n, "k": k,
                   "trans_a": False, "trans_b": False, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_FP32_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4), "traffic": traffic},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

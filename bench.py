#!/usr/bin/env python3
"""Benchmark of the fp32 GEMM hot path on one MI355X.

Default workload (BASELINE.json metric "fp32 GEMM TFLOP/s @4096^3"): nn::kernels::sgemm's replacement,
C = A B with A, B 4096 x 4096 fp32 from the reference's own seeded uniform[-1, 1] stream (seed 4, A filled
first, then B: apps/bench/runner.cpp:80-86). One step = one 4096^3 product; inputs are resident in HBM
before timing starts. Prints one JSON line on stdout (diagnostics go to stderr).

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

roofline.achieved = 2 M N K / (average kernel duration from HIP events recorded on the launch stream);
roofline.traffic comes from the committed rocprofv3 PMC summary (profiles/sgemm_4096_pmc.md) when present.
fused_op = the metric's "fused-op GB/s": conv2d_relu forward of config 3's memory-bound first layer.
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


def cpu_baseline(a, b, m, n, k, budget_s=15.0, max_runs=400):
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


def floor():
    """What a single launch costs on this GPU, beside the conv1 figure: an empty one-wave kernel (nnh.bench_delay
    with no delay), torch fills of conv1's output size (12.85 MB) and of eight times it, and copies of the same
    sizes, each timed as device_time_ms does. Prints a markdown table."""
    import torch

    import nnh
    dev = torch.device("cuda:0")
    ny = 128 * 32 * 784
    small, big = torch.empty(ny, device=dev), torch.empty(8 * ny, device=dev)
    src_small, src_big = torch.ones(ny // 2, device=dev), torch.ones(4 * ny, device=dev)
    rows = [("empty one-wave kernel (bench_delay 0)", lambda: nnh.bench_delay(0.0), 0),
            ("fill 12.85 MB (conv1's y)", lambda: small.fill_(1.0), 4 * ny),
            ("copy 6.4 MB -> 6.4 MB", lambda: small[: ny // 2].copy_(src_small), 4 * ny),
            ("fill 102.8 MB", lambda: big.fill_(1.0), 32 * ny),
            ("copy 51.4 MB -> 51.4 MB", lambda: big[: 4 * ny].copy_(src_big), 32 * ny)]
    print("| launch | us | GB/s | % of 8 TB/s |\n|---|---|---|---|")
    for name, fn, nbytes in rows:
        ms = device_time_ms(fn, reps=200)
        gbps = nbytes / (ms * 1e-3) / 1e9 if nbytes else 0.0
        print(f"| {name} | {ms * 1e3:.2f} | {gbps:.0f} | {gbps / PEAK_HBM_GBPS * 100:.1f}% |", flush=True)


def fused_op_conv1():
    """The metric's fused-op figure: nn::conv2d_relu forward of BASELINE config 3's first layer (x [128,1,28,28]
    U[0,1] seed 2, W [32,1,3,3] Kaiming-normal, zero bias, stride 1, pad 1), the memory-bound direct kernel
    with its bias/ReLU/alive epilogue. Algorithmic bytes: x + W + b read once, y written once (the alive flags
    are extra traffic, not counted). Device time from device_time_ms."""
    import numpy as np
    import torch

    import nnh
    from nnh import synth
    dev = torch.device("cuda:0")
    xc = synth.mt19937_uniform(2, 128 * 28 * 28, 0.0, 1.0).reshape(128, 1, 28, 28)
    w1 = (synth.normal(21, (32, 1, 3, 3)) * np.float32(np.sqrt(2.0 / 9))).astype(np.float32)
    dx, dw, db = (torch.from_numpy(np.ascontiguousarray(t)).to(dev) for t in (xc, w1, np.zeros(32, np.float32)))
    y = torch.empty((128, 32, 28, 28), device=dev)
    alive = torch.empty((128, 32, 28, 28), dtype=torch.uint8, device=dev)
    lib, stream = nnh.lib(), torch.cuda.current_stream()

    def step(al):
        nnh.check(lib.nnh_conv2d_forward(nnh._ptr(dx), 128, 1, 28, 28, nnh._ptr(dw), 32, 3, 3, nnh._ptr(db), 1, 1, 1,
                                         nnh._ptr(y), nnh._ptr(al), nnh._stream(stream)))

    nbytes = 4 * (xc.size + w1.size + 32 + y.numel())
    ms = device_time_ms(lambda: step(alive), reps=200)
    ms_no_alive = device_time_ms(lambda: step(None), reps=200)
    gbps = nbytes / (ms * 1e-3) / 1e9
    log(f"conv1 conv2d_relu: {ms * 1e3:.2f} us with alive flags ({gbps:.0f} GB/s), "
        f"{ms_no_alive * 1e3:.2f} us without")
    return {"workload": "conv2d_relu forward, BASELINE config 3 conv1: x [128,1,28,28] -> y [128,32,28,28], 3x3 s1 p1, "
                        "with alive flags", "value": round(gbps, 1), "unit": "GB/s", "us_per_launch": round(ms * 1e3, 3),
            "algorithmic_bytes": nbytes, "roofline": {"bound": "hbm", "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                                                      "frac": round(gbps / PEAK_HBM_GBPS, 4)},
            "without_alive_flags": {"us_per_launch": round(ms_no_alive * 1e3, 3),
                                    "value": round(nbytes / (ms_no_alive * 1e-3) / 1e9, 1)}}


# ---------------------------------------------------------------------------------------------------------------
# --report: every BASELINE.json config, absolute throughput and roofline fraction, nn-cpp's CPU path beside it

def device_time_ms(fn, reps=50, warmup_s=0.05, stream=None):
    """Average device time of one fn() (one or more launches on torch's current stream), without the
    Python caller's issue time: a bounded device-side delay (nnh.bench_delay) holds the stream while the
    host queues `reps` calls, then HIP events recorded on that stream around the calls time them back to
    back. Warm-up runs fn() for at least warmup_s of wall time so the clocks have ramped."""
    import torch

    import nnh
    stream = stream or torch.cuda.current_stream()
    t_end = time.perf_counter() + warmup_s
    n = 0
    while n < 3 or time.perf_counter() < t_end:
        fn()
        n += 1
    torch.cuda.synchronize()
    h0 = time.perf_counter()
    for _ in range(10):
        fn()
    issue_per_call = (time.perf_counter() - h0) / 10
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for attempt in range(5):
        delay_us = min(1.5e6, 1000.0 + 3.0 * reps * issue_per_call * 1e6)
        nnh.bench_delay(delay_us, stream)
        e0.record(stream)
        h0 = time.perf_counter()
        for _ in range(reps):
            fn()
        issued = time.perf_counter() - h0
        e1.record(stream)
        torch.cuda.synchronize()
        if issued * 1e6 <= delay_us:
            break
        # The host fell behind the delay (a long queue of launches and stream-ordered allocations behind a held
        # stream slows the caller down), so the events also timed host gaps: measure again with fewer calls.
        issue_per_call = issued / reps
        reps = max(4, reps // 4)
    else:
        log(f"  (host issue {issued * 1e6:.0f} us outlasted the {delay_us:.0f} us delay: the time includes host gaps)")
    return e0.elapsed_time(e1) / reps


def _cpu_time_ms(fn, budget_s=3.0, max_runs=15):
    """nn-cpp's method (apps/bench/runner.cpp:80-96): a warm-up, then the median of timed runs (bounded)."""
    fn()
    times, t_start = [], time.perf_counter()
    while len(times) < max_runs and (time.perf_counter() - t_start) < budget_s:
        t0 = time.perf_counter()
        fn()
        times.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(times)


U32 = 2.0 ** -24  # unit roundoff of fp32


def _host(t):
    return t.detach().cpu().numpy()


def _repeat_runs(run, times=3):
    """Runs the op `times` times (run() returns its output tensors); whether every run left the same bits, and the
    outputs of the first run on the host."""
    import numpy as np
    import torch
    first, same = None, True
    for _ in range(times):
        outs = run()
        torch.cuda.synchronize()
        cur = [np.array(_host(t), copy=True) for t in outs]
        if first is None:
            first = cur
        else:
            same = same and all(np.array_equal(a.view(np.uint32), b.view(np.uint32)) for a, b in zip(first, cur))
    return same, first


def _vs_cpu(got, want):
    """Largest |GPU - nn-cpp| over the outputs, and whether every bit agrees."""
    import numpy as np
    bitwise = all(np.array_equal(g.view(np.uint32), w.view(np.uint32)) for g, w in zip(got, want))
    diff = max(float(np.max(np.abs(g.astype(np.float64) - w.astype(np.float64)))) if g.size else 0.0
               for g, w in zip(got, want))
    return diff, bitwise


def _vs_f64(got, want, mag=None, terms=None):
    """Largest |GPU - fp64| and, given the magnitude sum mag = sum |a||b| and the number of product terms per
    output, the largest error as a fraction of the a-priori bound 4 terms 2^-24 mag (any summation order)."""
    import numpy as np
    err = np.abs(got.astype(np.float64) - want)
    worst = float(err.max()) if err.size else 0.0
    if mag is None:
        return worst, None
    bound = 4.0 * terms * U32 * mag
    ratio = np.where(bound > 0, err / np.where(bound > 0, bound, 1.0), np.where(err > 0, np.inf, 0.0))
    return worst, float(ratio.max()) if ratio.size else 0.0


def _conv_f64(x, w, b, pad):
    """Stride-1 convolution in fp64 and its magnitude sum, tap by tap."""
    import numpy as np
    N, C, H, W = x.shape
    O, _, kh, kw = w.shape
    ho, wo = H + 2 * pad - kh + 1, W + 2 * pad - kw + 1
    xp = np.pad(x.astype(np.float64), ((0, 0), (0, 0), (pad, pad), (pad, pad)))
    w64 = w.astype(np.float64)
    y = np.zeros((N, O, ho, wo))
    mag = np.zeros_like(y)
    for i in range(kh):
        for j in range(kw):
            win = xp[:, :, i:i + ho, j:j + wo]
            y += np.einsum("nchw,oc->nohw", win, w64[:, :, i, j], optimize=True)
            mag += np.einsum("nchw,oc->nohw", np.abs(win), np.abs(w64[:, :, i, j]), optimize=True)
    y += b.astype(np.float64)[None, :, None, None]
    mag += np.abs(b.astype(np.float64))[None, :, None, None]
    return y, mag


def _heads(t, heads):
    import numpy as np
    N, T, D = t.shape
    return t.astype(np.float64).reshape(N, T, heads, D // heads).transpose(0, 2, 1, 3)


def _attention_f64(q, k, v, g, heads, causal):
    """Attention forward (out) and backward (dq, dk, dv) in fp64, per head, with the softmax taken exactly."""
    import numpy as np
    N, T, D = q.shape
    scale = 1.0 / np.sqrt(D // heads)
    qh, kh, vh, gh = (_heads(t, heads) for t in (q, k, v, g))
    s = (qh @ kh.transpose(0, 1, 3, 2)) * scale
    if causal:
        s = np.where(np.triu(np.ones((T, k.shape[1]), bool), 1), -np.inf, s)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    merge = lambda t: t.transpose(0, 2, 1, 3).reshape(N, -1, D)
    out = merge(p @ vh)
    dp = gh @ vh.transpose(0, 1, 3, 2)
    ds = p * (dp - (dp * p).sum(-1, keepdims=True)) * scale
    return out, (merge(ds @ kh), merge(ds.transpose(0, 1, 3, 2) @ qh), merge(p.transpose(0, 1, 3, 2) @ gh))


def report(with_cpu=True):
    """Every BASELINE.json config on the GPU: time, TFLOP/s or GB/s, roofline fraction, nn-cpp's CPU time, and three
    checks of the outputs: bit equality over 3 repeated GPU runs, the largest difference from nn-cpp's CPU output
    on the same inputs (0 = bit for bit), and the largest error against fp64, also as a fraction of the bound
    4 K 2^-24 (|A||B|)_ij where the op is one product per output (K terms, any order)."""
    import numpy as np
    import torch

    import nnh
    from nnh import synth
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from pyoracle import Reference, reference_available
    ref = Reference() if (with_cpu and reference_available()) else None
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    if ref:
        ref.set_threads(threads)
    dev = torch.device("cuda:0")
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    rows = []

    def row(cfg, what, ms, flops=None, nbytes=None, bound="mfma", cpu_ms=None, repeat=None, cpu_diff=None,
            f64=None):
        tflops = flops / (ms * 1e-3) / 1e12 if flops else None
        gbps = nbytes / (ms * 1e-3) / 1e9 if nbytes else None
        frac = (tflops / PEAK_FP32_MFMA_TFLOPS) if bound == "mfma" else (gbps / PEAK_HBM_GBPS)
        rows.append({"config": cfg, "what": what, "ms": ms, "tflops": tflops, "gbps": gbps, "bound": bound,
                     "roofline_frac": frac, "cpu_ms": cpu_ms, "speedup_vs_cpu": (cpu_ms / ms) if cpu_ms else None,
                     "repeat": repeat, "cpu_diff": cpu_diff, "f64": f64})
        log(f"[{cfg}] {what}: {ms:.4f} ms" + (f", {tflops:.2f} TFLOP/s" if tflops else "") +
            (f", {gbps:.1f} GB/s" if gbps else "") + f", {frac * 100:.1f}% of {bound} peak" +
            (f"; nn-cpp CPU {cpu_ms:.3f} ms" if cpu_ms else "") +
            (f"; repeats bitwise {repeat}" if repeat is not None else "") +
            (f"; vs nn-cpp {cpu_diff[0]:.3g} (bitwise {cpu_diff[1]})" if cpu_diff else "") +
            (f"; vs fp64 {f64[0]:.3g}" + (f" = {f64[1]:.3g} of the bound" if f64[1] is not None else "")
             if f64 else ""))

    def worst(pairs):
        """Combines (abs error, fraction of bound) pairs over several outputs."""
        return (max(p[0] for p in pairs),
                None if any(p[1] is None for p in pairs) else max(p[1] for p in pairs))

    def gemm_f64(got, a, b, rows_of=None):
        """fp64 A B (on a sample of rows for large m) against the GPU's C."""
        a64, b64 = a.astype(np.float64), b.astype(np.float64)
        if rows_of is not None:
            a64, got = a64[rows_of], got[rows_of]
        return _vs_f64(got, a64 @ b64, np.abs(a64) @ np.abs(b64), a.shape[1])

    # config 1: 512^3, NN / TN / NT, seed 0
    n = 512
    a, b = synth.uniform_operands(0, [(n, n), (n, n)])
    da, db, dc = d(a), d(b), torch.empty((n, n), device=dev)
    c = np.empty((n, n), np.float32)
    for ta, tb, name in ((0, 0, "C=A B"), (1, 0, "C=A^T B"), (0, 1, "C=A B^T")):
        run = lambda: nnh.sgemm(ta, tb, n, n, n, da, n, db, n, dc, n)
        ms = device_time_ms(run)
        cpu = _cpu_time_ms(lambda: ref.sgemm_inplace(ta, tb, n, n, n, a, n, b, n, c, n, 0)) if ref else None
        same, (got,) = _repeat_runs(lambda: (run(), dc)[1:])
        row(1, f"sgemm 512^3 {name}", ms, flops=2.0 * n ** 3, cpu_ms=cpu, repeat=same,
            cpu_diff=_vs_cpu([got], [c]) if ref else None,
            f64=gemm_f64(got, a.T if ta else a, b.T if tb else b))

    # config 2: MLP 256 x 784 -> 512 -> 256 -> 10, forward (linear + ReLU) and backward (dX, dW, db)
    dims = [784, 512, 256, 10]
    x = synth.mt19937_uniform(1, 256 * 784, 0.0, 1.0).reshape(256, 784)
    ws = [synth.mt19937_uniform(100 + i, dims[i + 1] * dims[i], -1 / np.sqrt(dims[i]), 1 / np.sqrt(dims[i]))
          .reshape(dims[i + 1], dims[i]) for i in range(3)]
    bs = [np.zeros(dims[i + 1], np.float32) for i in range(3)]
    gys = [synth.normal(200 + i, (256, dims[i + 1])) for i in range(3)]
    dws, dbs, dgs = [d(w) for w in ws], [d(bb) for bb in bs], [d(g) for g in gys]
    acts = [d(x)]
    for i in range(3):
        acts.append(nnh.linear_forward(acts[-1], dws[i], dbs[i], relu=True))
    grads = [(torch.empty((256, dims[i]), device=dev), torch.empty(ws[i].shape, device=dev),
              torch.empty(dims[i + 1], device=dev)) for i in range(3)]

    def mlp_fwd():
        h, hs = acts[0], []
        for i in range(3):
            h = nnh.linear_forward(h, dws[i], dbs[i], relu=True)
            hs.append(h)
        return hs

    def mlp_bwd():
        for i in range(3):
            nnh.linear_backward(dgs[i], acts[i], dws[i], *[v for pair in zip(grads[i], (True,) * 3) for v in pair])
        return [t for gr in grads for t in gr]

    fwd_flops = sum(2.0 * 256 * dims[i] * dims[i + 1] for i in range(3))
    cpu, hacts = None, [x]
    if ref:
        for i in range(3):
            hacts.append(np.maximum(ref.linear_forward(hacts[-1], ws[i], bs[i]), np.float32(0)))

        def cpu_fwd():
            h = x
            for i in range(3):
                h = np.maximum(ref.linear_forward(h, ws[i], bs[i]), np.float32(0))
        cpu = _cpu_time_ms(cpu_fwd)
    ms = device_time_ms(mlp_fwd)
    same, hs = _repeat_runs(mlp_fwd)
    # each layer against fp64 from the GPU's own input to it (ReLU is 1-Lipschitz; the bias is one more term)
    ins = [x] + hs[:2]
    f64 = worst([_vs_f64(hs[i], np.maximum(ins[i].astype(np.float64) @ ws[i].T.astype(np.float64) + bs[i], 0),
                         np.abs(ins[i].astype(np.float64)) @ np.abs(ws[i].T.astype(np.float64)) + np.abs(bs[i]),
                         dims[i] + 1) for i in range(3)])
    row(2, "MLP forward (3 x linear+ReLU)", ms, flops=fwd_flops, cpu_ms=cpu, repeat=same,
        cpu_diff=_vs_cpu(hs, hacts[1:]) if ref else None, f64=f64)
    cpu, want = None, None
    if ref:
        want = [t for i in range(3) for t in ref.linear_backward(hacts[i], ws[i], bs[i], gys[i])]
        cpu = _cpu_time_ms(lambda: [ref.linear_backward(hacts[i], ws[i], bs[i], gys[i]) for i in range(3)])
    ms = device_time_ms(mlp_bwd)
    same, got = _repeat_runs(mlp_bwd)
    pairs = []
    for i in range(3):
        g64, x64, w64 = gys[i].astype(np.float64), _host(acts[i]).astype(np.float64), ws[i].astype(np.float64)
        pairs += [_vs_f64(got[3 * i], g64 @ w64, np.abs(g64) @ np.abs(w64), dims[i + 1]),
                  _vs_f64(got[3 * i + 1], g64.T @ x64, np.abs(g64.T) @ np.abs(x64), 256),
                  _vs_f64(got[3 * i + 2], g64.sum(0), np.abs(g64).sum(0), 256)]
    row(2, "MLP backward (dX, dW, db per layer)", ms, flops=2 * fwd_flops, cpu_ms=cpu, repeat=same,
        cpu_diff=_vs_cpu(got, want) if ref else None, f64=worst(pairs))

    # config 3: conv2d_relu, batch 128: conv1 1->32 on 28x28 (memory-bound), conv2 32->64 on 14x14
    xc = synth.mt19937_uniform(2, 128 * 28 * 28, 0.0, 1.0).reshape(128, 1, 28, 28)
    w1 = (synth.normal(21, (32, 1, 3, 3)) * np.float32(np.sqrt(2.0 / 9))).astype(np.float32)
    w2 = (synth.normal(22, (64, 32, 3, 3)) * np.float32(np.sqrt(2.0 / 288))).astype(np.float32)
    b1, b2 = np.zeros(32, np.float32), np.zeros(64, np.float32)
    dxc, dw1, dw2, db1, db2 = d(xc), d(w1), d(w2), d(b1), d(b2)
    y1, al1 = nnh.conv2d_forward(dxc, dw1, db1, 1, 1, True)
    x2 = torch.nn.functional.max_pool2d(y1, 2).contiguous()
    hx2 = x2.cpu().numpy()

    def conv_checks(run, x_, w_, b_, terms):
        same, (got,) = _repeat_runs(run)
        y64, mag = _conv_f64(x_, w_, b_, 1)
        cmp = _vs_cpu([got], [ref.conv2d_forward(x_, w_, b_, 1, 1, 1)]) if ref else None
        return dict(repeat=same, cpu_diff=cmp, f64=_vs_f64(got, np.maximum(y64, 0), mag, terms))

    conv1_bytes = 4 * (xc.size + w1.size + b1.size + 128 * 32 * 784)
    cpu = _cpu_time_ms(lambda: ref.conv2d_forward(xc, w1, b1, 1, 1, 1)) if ref else None
    run = lambda: nnh.conv2d_forward(dxc, dw1, db1, 1, 1, True)
    row(3, "conv1 conv2d_relu fwd (1->32, 28x28, b128)", device_time_ms(run),
        flops=2.0 * 128 * 32 * 784 * 9, nbytes=conv1_bytes, bound="hbm", cpu_ms=cpu,
        **conv_checks(lambda: run()[:1], xc, w1, b1, 10))
    run = lambda: nnh.conv2d_forward(dxc, dw1, db1, 1, 1, True, want_alive=False)
    row(3, "conv1 conv2d_relu fwd, no alive flags (backward masks with y > 0)", device_time_ms(run),
        flops=2.0 * 128 * 32 * 784 * 9, nbytes=conv1_bytes, bound="hbm",
        **conv_checks(lambda: run()[:1], xc, w1, b1, 10))
    # not a BASELINE config: the same layer at batch 2048 shows the kernel's streaming rate once launch and
    # drain latency (about 4 us for any 13 MB launch on this GPU) no longer dominate
    xbig = dxc.repeat(16, 1, 1, 1)
    row("3*", "conv1 conv2d_relu fwd at batch 2048 (steady state)",
        device_time_ms(lambda: nnh.conv2d_forward(xbig, dw1, db1, 1, 1, True), reps=20),
        flops=16 * 2.0 * 128 * 32 * 784 * 9, nbytes=16 * (conv1_bytes - 4 * (w1.size + b1.size)) + 4 * (w1.size + b1.size),
        bound="hbm")
    del xbig
    cpu = _cpu_time_ms(lambda: ref.conv2d_forward(hx2, w2, b2, 1, 1, 1)) if ref else None
    run = lambda: nnh.conv2d_forward(x2, dw2, db2, 1, 1, True)
    row(3, "conv2 conv2d_relu fwd (32->64, 14x14, b128)", device_time_ms(run),
        flops=2.0 * 128 * 64 * 196 * 288, nbytes=4 * (hx2.size + w2.size + 64 + 128 * 64 * 196), cpu_ms=cpu,
        **conv_checks(lambda: run()[:1], hx2, w2, b2, 289))
    y2, al2 = nnh.conv2d_forward(x2, dw2, db2, 1, 1, True)
    hg2 = synth.normal(32, tuple(y2.shape))
    g2 = d(hg2)
    gx2, gw2, gb2 = torch.empty_like(x2), torch.empty_like(dw2), torch.empty_like(db2)
    cpu, want = None, None
    if ref:
        want = list(ref.conv2d_backward(hx2, w2, b2, 1, 1, 1, hg2))
        cpu = _cpu_time_ms(lambda: ref.conv2d_backward(hx2, w2, b2, 1, 1, 1, hg2))
    run = lambda: nnh.conv2d_backward(g2, x2, dw2, al2, 1, 1, gx2, True, gw2, True, gb2, True)
    ms = device_time_ms(run)
    same, got = _repeat_runs(lambda: (run(), gx2, gw2, gb2)[1:])
    # fp64 gradients of the masked output gradient gm: dx is the transposed convolution (Cout kh kw terms),
    # dW correlates gm with the padded input (N Ho Wo terms), db sums gm
    gm = hg2.astype(np.float64) * (_host(y2) > 0)
    xp = np.pad(hx2.astype(np.float64), ((0, 0), (0, 0), (1, 1), (1, 1)))
    dx64, dxmag = np.zeros(xp.shape), np.zeros(xp.shape)
    dw64, dwmag = np.zeros(w2.shape), np.zeros(w2.shape)
    for i in range(3):
        for j in range(3):
            win = xp[:, :, i:i + 14, j:j + 14]
            dw64[:, :, i, j] = np.einsum("nohw,nchw->oc", gm, win, optimize=True)
            dwmag[:, :, i, j] = np.einsum("nohw,nchw->oc", np.abs(gm), np.abs(win), optimize=True)
            dx64[:, :, i:i + 14, j:j + 14] += np.einsum("nohw,oc->nchw", gm, w2[:, :, i, j].astype(np.float64),
                                                        optimize=True)
            dxmag[:, :, i:i + 14, j:j + 14] += np.einsum("nohw,oc->nchw", np.abs(gm),
                                                         np.abs(w2[:, :, i, j].astype(np.float64)), optimize=True)
    f64 = worst([_vs_f64(got[0], dx64[:, :, 1:15, 1:15], dxmag[:, :, 1:15, 1:15], 64 * 9),
                 _vs_f64(got[1], dw64, dwmag, 128 * 196),
                 _vs_f64(got[2], gm.sum((0, 2, 3)), np.abs(gm).sum((0, 2, 3)), 128 * 196)])
    row(3, "conv2 conv2d_relu bwd (dx, dW, db)", ms, flops=2 * 2.0 * 128 * 64 * 196 * 288, cpu_ms=cpu,
        repeat=same, cpu_diff=_vs_cpu(got, want) if ref else None, f64=f64)

    # config 4: attention 32 x 8 heads x 256 x 64 (+ causal); probs stored, as the reference does
    q, k, v = (synth.normal(3 + i, (32, 256, 512)) for i in range(3))
    hg = synth.normal(7, (32, 256, 512))
    dq_, dk_, dv_ = d(q), d(k), d(v)
    att_flops = 2 * 2.0 * 32 * 8 * 256 * 256 * 64
    out64, grads64 = _attention_f64(q, k, v, hg, 8, False)
    for causal in (False, True):
        cpu = _cpu_time_ms(lambda: ref.attention_forward(q, k, v, 8, None, causal), budget_s=4.0, max_runs=5) if ref else None
        run = lambda: nnh.attention_forward(dq_, dk_, dv_, 8, None, causal)
        ms = device_time_ms(run)
        same, (got,) = _repeat_runs(lambda: run()[:1])
        want64 = out64 if not causal else _attention_f64(q, k, v, hg, 8, True)[0]
        row(4, "attention fwd" + (" causal" if causal else ""), ms, flops=att_flops, cpu_ms=cpu, repeat=same,
            cpu_diff=_vs_cpu([got], [ref.attention_forward(q, k, v, 8, None, causal)]) if ref else None,
            f64=_vs_f64(got, want64))
    out, probs = nnh.attention_forward(dq_, dk_, dv_, 8, None, False)
    ga = d(hg)
    gq, gk, gv = torch.empty_like(dq_), torch.empty_like(dk_), torch.empty_like(dv_)
    cpu, want = None, None
    if ref:
        want = list(ref.attention_backward(q, k, v, 8, hg))
        cpu = _cpu_time_ms(lambda: ref.attention_backward(q, k, v, 8, hg), budget_s=4.0, max_runs=3)
    run = lambda: nnh.attention_backward(ga, dq_, dk_, dv_, probs, 8, None, False, gq, True, gk, True, gv, True)
    ms = device_time_ms(run)
    same, got = _repeat_runs(lambda: (run(), gq, gk, gv)[1:])
    row(4, "attention bwd (dQ, dK, dV)", ms, flops=2 * att_flops, cpu_ms=cpu, repeat=same,
        cpu_diff=_vs_cpu(got, want) if ref else None, f64=worst([_vs_f64(g_, w_) for g_, w_ in zip(got, grads64)]))
    del out64, grads64

    # config 5: roofline sweep, seed 4; fp64 on 256 evenly spaced rows when m >= 2048
    for (m, n_, k_) in ((1024, 1024, 1024), (2048, 2048, 2048), (4096, 4096, 4096), (8192, 8192, 8192),
                        (64, 4096, 4096), (4096, 4096, 64)):
        a, b = synth.uniform_operands(4, [(m, k_), (k_, n_)])
        da, db, dc = d(a), d(b), torch.empty((m, n_), device=dev)
        c = np.empty((m, n_), np.float32)
        reps = 5 if m * n_ * k_ >= 8192 ** 3 else 20
        cpu = _cpu_time_ms(lambda: ref.sgemm_inplace(0, 0, m, n_, k_, a, k_, b, n_, c, n_, 0),
                           budget_s=6.0, max_runs=5) if ref else None
        run = lambda: nnh.sgemm(0, 0, m, n_, k_, da, k_, db, n_, dc, n_)
        ms = device_time_ms(run, reps=reps)
        same, (got,) = _repeat_runs(lambda: (run(), dc)[1:])
        sample = np.linspace(0, m - 1, 256).astype(np.int64) if m >= 2048 else None
        row(5, f"sgemm {m}x{n_}x{k_}", ms, flops=2.0 * m * n_ * k_, cpu_ms=cpu, repeat=same,
            cpu_diff=_vs_cpu([got], [c]) if ref else None, f64=gemm_f64(got, a, b, sample))
        del got, c

    lines = [f"GPU: {torch.cuda.get_device_name(0)}; nn-cpp CPU baseline: NN_NATIVE AVX2 build, {threads} threads on "
             f"{cpu_model()}", "",
             "| cfg | workload | GPU ms | TFLOP/s | GB/s | bound | % of roofline | nn-cpp CPU ms | GPU speedup | "
             "3 GPU runs | max abs diff vs nn-cpp | max abs err vs fp64 | err / bound |",
             "|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for r in rows:
        f = lambda v, fmt: (fmt % v) if v is not None else "-"
        rep = "-" if r["repeat"] is None else ("bitwise equal" if r["repeat"] else "DIFFER")
        cd = "-" if r["cpu_diff"] is None else ("0 (bitwise)" if r["cpu_diff"][1] else "%.3g" % r["cpu_diff"][0])
        fe = r["f64"] or (None, None)
        lines.append(f"| {r['config']} | {r['what']} | {r['ms']:.4f} | {f(r['tflops'], '%.2f')} | {f(r['gbps'], '%.0f')} | "
                     f"{r['bound']} | {r['roofline_frac'] * 100:.1f}% | {f(r['cpu_ms'], '%.3f')} | "
                     f"{f(r['speedup_vs_cpu'], '%.0fx')} | {rep} | {cd} | {f(fe[0], '%.3g')} | {f(fe[1], '%.3g')} |")
    print("\n".join(lines), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--size", type=int, default=4096)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-fused-op", action="store_true", help="skip the conv1 fused conv2d_relu GB/s figure")
    ap.add_argument("--report", action="store_true", help="every BASELINE config as a markdown table (not the "
                    "driver's JSON line)")
    ap.add_argument("--floor", action="store_true", help="launch-cost floor of this GPU: empty kernel, fills, copies")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run 5 device-to-device copies of MIB MiB (calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); --gpus {args.gpus} is not "
              "supported", file=sys.stderr)
        sys.exit(2)
    if args.report:
        report(with_cpu=not args.no_cpu_baseline)
        return
    if args.floor:
        floor()
        return
    if args.copy_probe:
        import torch
        nbytes = args.copy_probe << 20
        src = torch.ones(nbytes // 4, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: 5 copies of {nbytes} bytes ({nbytes / 1024:.0f} KiB read + written per copy)")
        return

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

    fused = None if args.no_fused_op else fused_op_conv1()
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
        "fused_op": fused,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

#!/usr/bin/env python3
"""Benchmark of nn-cpp's fp32 GEMM hot path on one MI355X.

The JSON line's headline (BASELINE.json metric "fp32 GEMM TFLOP/s @4096^3"): nn::kernels::sgemm's replacement,
C = A B with A, B 4096 x 4096 fp32 from the reference's own seeded uniform[-1, 1] stream (seed 4, A filled first,
then B: apps/bench/runner.cpp:80-86). One step = one 4096^3 product; inputs are resident in HBM before timing
starts. Before the W warm-up steps the clock is settled with launches for at least SETTLE_S seconds (it ramps
over the first ~20 launches), reported as settle_launches.

`configs` holds every BASELINE.json configuration (cfg 1-5) as rows: the op's median device time over BATCHES
batches of back-to-back calls (stats.hpp:24-58's median and IQR/median spread), TFLOP/s or GB/s, its roofline
fraction, whether three GPU runs and nn-cpp's own CPU output agree bit for bit, and nn-cpp's CPU time for the same
op on the same host buffers (the reference's NN_NATIVE AVX2 build, oracle/_ref, timed in C++ as runner.cpp does:
nn::matmul for configs 1 and 5, linear + relu for 2, conv2d_relu for 3, attention for 4; backward rows time the
op's own backward rule), on one thread per physical core of the cores this process may use, pinned, and on one
thread. Prints one JSON line on stdout (diagnostics go to stderr).

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-configs] [--csv PATH]
  python bench.py --report      # the same rows as a markdown table, with fp64 error bounds
  python bench.py --floor       # launch-cost floor of this GPU
"""
import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "nn-cpp_amd"))

PEAK_FP32_MFMA_TFLOPS = 157.3   # MI355X dense fp32 matrix peak (AMD spec)
PEAK_HBM_GBPS = 8000.0          # MI355X HBM3E
SETTLE_S = 0.5                  # clock settling before the headline's warm-up
BATCHES = 7                     # timed batches per config row (median and spread over them)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def traffic_from_profile(name):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, copy-calibrated)."""
    path = os.path.join(ROOT, "profiles", f"{name}_pmc.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"hbm_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read())
    return float(m.group(1)) if m else None


# ---------------------------------------------------------------------------------------------------------------
# statistics: apps/bench/stats.hpp (linear-interpolated quantiles)

def quantile_sorted(s, q):
    pos = q * (len(s) - 1)
    lo = int(pos)
    hi = min(lo + 1, len(s) - 1)
    return s[lo] + (pos - lo) * (s[hi] - s[lo])


def median(v):
    return quantile_sorted(sorted(v), 0.5)


def spread(v):
    if len(v) < 2:
        return 0.0
    s = sorted(v)
    return (quantile_sorted(s, 0.75) - quantile_sorted(s, 0.25)) / quantile_sorted(s, 0.5)


# ---------------------------------------------------------------------------------------------------------------
# the host CPU (for the baseline): model, governor, one logical CPU per physical core

def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def cpu_governor():
    try:
        return open("/sys/devices/system/cpu/cpu0/cpufreq/scaling_governor").read().strip()
    except OSError:
        return "unknown"


def physical_cores():
    """One logical CPU per physical core among the CPUs this process may run on, and the allowed CPU count."""
    allowed = sorted(os.sched_getaffinity(0))
    first = {}
    for c in allowed:
        base = f"/sys/devices/system/cpu/cpu{c}/topology/"
        try:
            key = (int(open(base + "physical_package_id").read()), int(open(base + "core_id").read()))
        except (OSError, ValueError):
            key = (0, c)
        first.setdefault(key, c)
    return sorted(first.values()), len(allowed)


# ---------------------------------------------------------------------------------------------------------------
# device timing

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


def device_times(fn, est_ms):
    """BATCHES device-time measurements of fn (each an average over back-to-back calls); the first also warms up."""
    reps = int(max(4, min(100, 20.0 / max(est_ms, 1e-3))))
    out = [device_time_ms(fn, reps=reps, warmup_s=0.1)]
    for _ in range(BATCHES - 1):
        out.append(device_time_ms(fn, reps=reps, warmup_s=0.0))
    return out


# ---------------------------------------------------------------------------------------------------------------
# fp64 checks (--report)

U32 = 2.0 ** -24  # unit roundoff of fp32


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


def _worst(pairs):
    return (max(p[0] for p in pairs), None if any(p[1] is None for p in pairs) else max(p[1] for p in pairs))


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


def _conv_bwd_f64(gm, x, w):
    """fp64 gradients of a stride-1, padding-1 3x3 convolution for the masked output gradient gm: dx (Cout kh kw
    terms), dW (N Ho Wo terms), db, each with its magnitude sum."""
    import numpy as np
    _, _, H, W = x.shape
    xp = np.pad(x.astype(np.float64), ((0, 0), (0, 0), (1, 1), (1, 1)))
    dx64, dxmag = np.zeros(xp.shape), np.zeros(xp.shape)
    dw64, dwmag = np.zeros(w.shape), np.zeros(w.shape)
    for i in range(3):
        for j in range(3):
            win = xp[:, :, i:i + H, j:j + W]
            w64 = w[:, :, i, j].astype(np.float64)
            dw64[:, :, i, j] = np.einsum("nohw,nchw->oc", gm, win, optimize=True)
            dwmag[:, :, i, j] = np.einsum("nohw,nchw->oc", np.abs(gm), np.abs(win), optimize=True)
            dx64[:, :, i:i + H, j:j + W] += np.einsum("nohw,oc->nchw", gm, w64, optimize=True)
            dxmag[:, :, i:i + H, j:j + W] += np.einsum("nohw,oc->nchw", np.abs(gm), np.abs(w64), optimize=True)
    return ((dx64[:, :, 1:H + 1, 1:W + 1], dxmag[:, :, 1:H + 1, 1:W + 1]), (dw64, dwmag),
            (gm.sum((0, 2, 3)), np.abs(gm).sum((0, 2, 3))))


def _attention_f64(q, k, v, g, heads, causal):
    """Attention forward (out) and backward (dq, dk, dv) in fp64, per head, with the softmax taken exactly."""
    import numpy as np
    N, T, D = q.shape
    scale = 1.0 / np.sqrt(D // heads)
    hd = lambda t: t.astype(np.float64).reshape(N, T, heads, D // heads).transpose(0, 2, 1, 3)
    qh, kh, vh, gh = hd(q), hd(k), hd(v), hd(g)
    s = (qh @ kh.transpose(0, 1, 3, 2)) * scale
    if causal:
        s = np.where(np.triu(np.ones((T, T), bool), 1), -np.inf, s)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    merge = lambda t: t.transpose(0, 2, 1, 3).reshape(N, -1, D)
    dp = gh @ vh.transpose(0, 1, 3, 2)
    ds = p * (dp - (dp * p).sum(-1, keepdims=True)) * scale
    return merge(p @ vh), (merge(ds @ kh), merge(ds.transpose(0, 1, 3, 2) @ qh), merge(p.transpose(0, 1, 3, 2) @ gh))


# ---------------------------------------------------------------------------------------------------------------
# the BASELINE.json configurations as rows

class Row:
    """One measured op. gpu() launches it once on device-resident inputs (writing fixed outputs); outs() returns
    those output tensors; cpu(ref, warmup, runs, budget) times nn-cpp's own op on the same host buffers and returns
    (times_ms, outputs); f64(host_outs) gives (max abs error vs fp64, fraction of the error bound)."""

    def __init__(self, cfg, key, workload, gpu, outs, flops, nbytes=None, bound="mfma", cpu=None, f64=None,
                 est_ms=0.05, useful_flops=None):
        self.cfg, self.key, self.workload = cfg, key, workload
        self.gpu, self.outs, self.cpu, self.f64 = gpu, outs, cpu, f64
        self.flops, self.nbytes, self.bound, self.est_ms, self.useful_flops = flops, nbytes, bound, est_ms, useful_flops
        self.result = {}


def build_rows(report=False, split=False):
    """Inputs of every BASELINE.json configuration (the reference's seeded streams), resident on the GPU, and one
    Row per measured op (split: only the GEMM-shaped rows of configs 1, 2 and 5 that the split-depth mode changes,
    to be run in that mode)."""
    import ctypes as C

    import numpy as np
    import torch

    import nnh
    from nnh import synth
    L = nnh.lib()
    dev = torch.device("cuda:0")
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    st = lambda: nnh._stream(None)
    P = nnh._ptr
    rows = []

    def shape_arr(s):
        return (C.c_size_t * len(s))(*s)

    def matmul_row(cfg, key, what, seed, m, n, k, ta, tb, est_ms):
        a, b = synth.uniform_operands(seed, [(k, m) if ta else (m, k), (n, k) if tb else (k, n)])
        da, db = d(a), d(b)
        dc = torch.empty((m, n), device=dev)
        ash, bsh = shape_arr(a.shape), shape_arr(b.shape)

        def gpu():
            nnh.check(L.nnh_matmul(P(da), ash, 2, P(db), bsh, 2, ta, tb, P(dc), st()))

        def f64(h):
            a64 = (a.T if ta else a).astype(np.float64)
            b64 = (b.T if tb else b).astype(np.float64)
            rows_of = np.linspace(0, m - 1, 256).astype(np.int64) if m >= 2048 else slice(None)
            return _vs_f64(h[0][rows_of], a64[rows_of] @ b64, np.abs(a64[rows_of]) @ np.abs(b64), k)

        rows.append(Row(cfg, key, what, gpu, lambda: [dc], 2.0 * m * n * k,
                        cpu=lambda ref, w, r, bud: (lambda t, o: (t, [o]))(*ref.time_matmul(a, b, ta, tb, w, r, bud)),
                        f64=f64, est_ms=est_ms))

    # config 1: 512^3 through nn::matmul, C = A B, A^T B, A B^T (seed 0)
    for ta, tb, name in ((0, 0, "A B"), (1, 0, "A^T B"), (0, 1, "A B^T")):
        matmul_row(1, f"matmul512_{'t' if ta else 'n'}{'t' if tb else 'n'}", f"nn::matmul 512^3 C = {name}", 0,
                   512, 512, 512, ta, tb, 0.01)

    # config 2: MLP 256 x 784 -> 512 -> 256 -> 10, linear + ReLU per layer; backward dX, dW, db per layer (seed 1)
    dims = [784, 512, 256, 10]
    M = 256
    x = synth.mt19937_uniform(1, M * 784, 0.0, 1.0).reshape(M, 784)
    ws = [synth.mt19937_uniform(100 + i, dims[i + 1] * dims[i], -1 / np.sqrt(dims[i]), 1 / np.sqrt(dims[i]))
          .reshape(dims[i + 1], dims[i]) for i in range(3)]
    bs = [np.zeros(dims[i + 1], np.float32) for i in range(3)]
    gys = [synth.normal(200 + i, (M, dims[i + 1])) for i in range(3)]
    dws, dbs, dgs = [d(w) for w in ws], [d(b) for b in bs], [d(g) for g in gys]
    acts = [d(x)] + [torch.empty((M, dims[i + 1]), device=dev) for i in range(3)]
    grads = [(torch.empty((M, dims[i]), device=dev), torch.empty(ws[i].shape, device=dev),
              torch.empty(dims[i + 1], device=dev)) for i in range(3)]
    lead = shape_arr([M])

    def mlp_fwd():
        for i in range(3):
            nnh.check(L.nnh_linear_forward(P(acts[i]), M, dims[i], P(dws[i]), dims[i + 1], P(dbs[i]), 1, P(acts[i + 1]),
                                           st()))

    mlp_fwd()
    hacts = [x] + [acts[i + 1].cpu().numpy() for i in range(3)]

    def mlp_bwd():
        for i in range(3):
            nnh.check(L.nnh_linear_backward(P(dgs[i]), P(acts[i]), P(dws[i]), lead, 1, dims[i], dims[i + 1],
                                            P(grads[i][0]), 1, P(grads[i][1]), 1, P(grads[i][2]), 1, st()))

    def mlp_fwd_f64(h):
        ins = [x] + h[:2]
        return _worst([_vs_f64(h[i], np.maximum(ins[i].astype(np.float64) @ ws[i].T.astype(np.float64) + bs[i], 0),
                               np.abs(ins[i].astype(np.float64)) @ np.abs(ws[i].T.astype(np.float64)) + np.abs(bs[i]),
                               dims[i] + 1) for i in range(3)])

    def mlp_bwd_f64(h):
        pairs = []
        for i in range(3):
            g64, x64, w64 = gys[i].astype(np.float64), hacts[i].astype(np.float64), ws[i].astype(np.float64)
            pairs += [_vs_f64(h[3 * i], g64 @ w64, np.abs(g64) @ np.abs(w64), dims[i + 1]),
                      _vs_f64(h[3 * i + 1], g64.T @ x64, np.abs(g64.T) @ np.abs(x64), M),
                      _vs_f64(h[3 * i + 2], g64.sum(0), np.abs(g64).sum(0), M)]
        return _worst(pairs)

    fwd_flops = sum(2.0 * M * dims[i] * dims[i + 1] for i in range(3))
    rows.append(Row(2, "mlp_forward", "MLP forward: 3 x nn::linear + ReLU, 256 x 784 -> 512 -> 256 -> 10", mlp_fwd,
                    lambda: acts[1:], fwd_flops,
                    cpu=lambda ref, w, r, bud: ref.time_linear_relu_chain(x, ws, bs, w, r, bud), f64=mlp_fwd_f64,
                    est_ms=0.03))
    rows.append(Row(2, "mlp_backward", "MLP backward: nn::linear's dX, dW, db for each of the 3 layers", mlp_bwd,
                    lambda: [t for gr in grads for t in gr], 2 * fwd_flops,
                    cpu=lambda ref, w, r, bud: ref.time_linear_backward_layers(hacts[:3], ws, bs, gys, w, r, bud),
                    f64=mlp_bwd_f64, est_ms=0.035))

    if split:  # the products the split-depth mode changes: configs 1 and 2 and the skinny config 5 product
        matmul_row(5, "matmul_64x4096x4096", "nn::matmul 64x4096x4096 C = A B", 4, 64, 4096, 4096, 0, 0, 0.06)
        for r in rows:
            r.key += "_split"
            r.workload += " [NNH_NUMERICS_SPLIT_DEPTH]"
            r.cpu = None
        return rows

    # config 3: conv2d_relu, batch 128: conv1 1 -> 32 on 28 x 28 (memory-bound), conv2 32 -> 64 on 14 x 14 after a
    # 2 x 2 max pool (seed 2)
    N = 128
    xc = synth.mt19937_uniform(2, N * 28 * 28, 0.0, 1.0).reshape(N, 1, 28, 28)
    w1 = (synth.normal(21, (32, 1, 3, 3)) * np.float32(np.sqrt(2.0 / 9))).astype(np.float32)
    w2 = (synth.normal(22, (64, 32, 3, 3)) * np.float32(np.sqrt(2.0 / 288))).astype(np.float32)
    b1, b2 = np.zeros(32, np.float32), np.zeros(64, np.float32)
    dxc, dw1, dw2, db1, db2 = d(xc), d(w1), d(w2), d(b1), d(b2)
    y1, al1 = torch.empty((N, 32, 28, 28), device=dev), torch.empty((N, 32, 28, 28), dtype=torch.uint8, device=dev)

    def conv_fwd(x_, w_, b_, y_, al_, dims_):
        n_, cin, h, w__ = dims_
        return lambda: nnh.check(L.nnh_conv2d_forward(P(x_), n_, cin, h, w__, P(w_), w_.shape[0], 3, 3, P(b_), 1, 1, 1,
                                                      P(y_), P(al_) if al_ is not None else None, st()))

    conv1 = conv_fwd(dxc, dw1, db1, y1, al1, (N, 1, 28, 28))
    conv1()
    x2 = torch.empty((N, 32, 14, 14), device=dev)
    arg1 = torch.empty((N, 32, 14, 14), dtype=torch.int32, device=dev)

    def pool1():
        nnh.check(L.nnh_maxpool2d_forward(P(y1), N, 32, 28, 28, 2, 2, P(x2), C.c_void_p(arg1.data_ptr()), st()))

    pool1()
    hx2 = x2.cpu().numpy()
    y2, al2 = torch.empty((N, 64, 14, 14), device=dev), torch.empty((N, 64, 14, 14), dtype=torch.uint8, device=dev)
    conv2 = conv_fwd(x2, dw2, db2, y2, al2, (N, 32, 14, 14))
    conv2()
    hy1, hy2 = y1.cpu().numpy(), y2.cpu().numpy()
    hg1, hg2 = synth.normal(31, (N, 32, 28, 28)), synth.normal(32, (N, 64, 14, 14))
    g1, g2 = d(hg1), d(hg2)
    gx1, gw1, gb1 = torch.empty_like(dxc), torch.empty_like(dw1), torch.empty_like(db1)
    gx2, gw2, gb2 = torch.empty_like(x2), torch.empty_like(dw2), torch.empty_like(db2)

    def conv_bwd(g_, x_, w_, al_, dims_, outs_):
        n_, cin, h, w__ = dims_
        gx, gw, gb = outs_
        return lambda: nnh.check(L.nnh_conv2d_backward(P(g_), P(x_), P(w_), P(al_), n_, cin, h, w__, w_.shape[0], 3, 3,
                                                       1, 1, P(gx), 1, P(gw), 1, P(gb), 1, st()))

    conv_cache = {}

    def conv_cpu(which, ref, w, r, bud):
        """nn-cpp's conv2d_relu forward and backward rule for one layer; both rows of a layer share one call."""
        if (which, w, r, bud) not in conv_cache:
            xx, ww, bb, gg = (xc, w1, b1, hg1) if which == 1 else (hx2, w2, b2, hg2)
            conv_cache[(which, w, r, bud)] = ref.time_conv2d(xx, ww, bb, 1, 1, 1, gg, w, r, bud)
        return conv_cache[(which, w, r, bud)]

    def conv_fwd_f64(x_, w_, b_, terms):
        return lambda h: (lambda y64, mag: _vs_f64(h[0], np.maximum(y64, 0), mag, terms))(*_conv_f64(x_, w_, b_, 1))

    def conv_bwd_f64(hg, hy, x_, w_, hw):
        def f(h):
            (dx64, dxm), (dw64, dwm), (db64, dbm) = _conv_bwd_f64(hg.astype(np.float64) * (hy > 0), x_, w_)
            return _worst([_vs_f64(h[0], dx64, dxm, w_.shape[0] * 9), _vs_f64(h[1], dw64, dwm, N * hw),
                           _vs_f64(h[2], db64, dbm, N * hw)])
        return f

    conv1_bytes = 4 * (xc.size + w1.size + b1.size + N * 32 * 784)
    conv1_flops = 2.0 * N * 32 * 784 * 9
    rows.append(Row(3, "conv1_forward", "conv2d_relu forward, conv1: x [128,1,28,28] -> y [128,32,28,28], 3x3 s1 p1, "
                    "with alive flags", conv1, lambda: [y1], conv1_flops, nbytes=conv1_bytes, bound="hbm",
                    cpu=lambda ref, w, r, bud: (lambda f, b: (f[0], [f[1]]))(*conv_cpu(1, ref, w, r, bud)),
                    f64=conv_fwd_f64(xc, w1, b1, 10), est_ms=0.006))
    conv1_na = conv_fwd(dxc, dw1, db1, y1, None, (N, 1, 28, 28))
    rows.append(Row(3, "conv1_forward_no_alive", "conv2d_relu forward, conv1, without alive flags (the backward masks "
                    "with y > 0)", conv1_na, lambda: [y1], conv1_flops, nbytes=conv1_bytes, bound="hbm",
                    f64=conv_fwd_f64(xc, w1, b1, 10), est_ms=0.006))
    conv1_bwd_bytes = 4 * (hg1.size + xc.size + w1.size + xc.size + w1.size + b1.size)
    rows.append(Row(3, "conv1_backward", "conv2d_relu backward, conv1: dx, dW, db (g masked by alive)",
                    conv_bwd(g1, dxc, dw1, al1, (N, 1, 28, 28), (gx1, gw1, gb1)), lambda: [gx1, gw1, gb1],
                    2 * conv1_flops, nbytes=conv1_bwd_bytes, bound="hbm",
                    cpu=lambda ref, w, r, bud: (lambda f, b: (b[0], list(b[1])))(*conv_cpu(1, ref, w, r, bud)),
                    f64=conv_bwd_f64(hg1, hy1, xc, w1, 784), est_ms=0.03))
    hy1c = y1.cpu().numpy()
    hgp = synth.normal(33, (N, 32, 14, 14))
    gp, gxp = d(hgp), torch.empty_like(y1)
    pool_cache = {}

    def pool_cpu(ref, w, r, bud):
        if (w, r, bud) not in pool_cache:
            pool_cache[(w, r, bud)] = ref.time_maxpool2d(hy1c, 2, 2, hgp, w, r, bud)
        return pool_cache[(w, r, bud)]

    def pool1_bwd():
        nnh.check(L.nnh_maxpool2d_backward(P(gp), C.c_void_p(arg1.data_ptr()), N, 32, 28, 28, 2, 2, P(gxp), 1, st()))

    pool_bytes = 4 * (hy1c.size + hx2.size)
    rows.append(Row(3, "pool1_forward", "maxpool2d forward 2x2 s2 on conv1's output: [128,32,28,28] -> [128,32,14,14]"
                    " (argmax kept)", pool1, lambda: [x2, arg1], 0, nbytes=pool_bytes, bound="hbm",
                    cpu=lambda ref, w, r, bud: (lambda f, b: (f[0], [f[1], None]))(*pool_cpu(ref, w, r, bud)),
                    est_ms=0.005))
    y1f, al1f = torch.empty_like(y1), torch.empty_like(al1)
    x2f, arg1f = torch.empty_like(x2), torch.empty_like(arg1)

    def conv1_pool1():
        nnh.check(L.nnh_conv2d_relu_maxpool2d_forward(P(dxc), N, 1, 28, 28, P(dw1), 32, 3, 3, P(db1), 1, 1, 2, 2,
                                                      P(y1f), P(al1f), P(x2f), C.c_void_p(arg1f.data_ptr()), st()))

    rows.append(Row(3, "conv1_pool1_forward", "conv2d_relu forward of conv1 and the 2x2 s2 maxpool on its output in one "
                    "pass: y [128,32,28,28] with alive flags, pooled [128,32,14,14] with argmax",
                    conv1_pool1, lambda: [y1f, al1f, x2f, arg1f], conv1_flops, nbytes=conv1_bytes + 4 * hx2.size,
                    bound="hbm", est_ms=0.007))
    rows.append(Row(3, "pool1_backward", "maxpool2d backward 2x2 s2: dx [128,32,28,28] from g [128,32,14,14]",
                    pool1_bwd, lambda: [gxp], 0, nbytes=pool_bytes, bound="hbm",
                    cpu=lambda ref, w, r, bud: (lambda f, b: (b[0], [b[1]]))(*pool_cpu(ref, w, r, bud)),
                    est_ms=0.008))
    # the packed forms (nnh.h): ReLU flags one bit per output, a pooled output's maximum as its 2-bit position in the
    # window; the same values and gradients as the byte forms above (checked bit for bit in main)
    y1p, bits1 = torch.empty_like(y1), torch.empty(N * 32 * 784 // 8, dtype=torch.uint8, device=dev)

    def conv1_packed():
        nnh.check(L.nnh_conv2d_relu_forward_packed(P(dxc), N, 1, 28, 28, P(dw1), 32, 3, 3, P(db1), 1, 1, P(y1p),
                                                   P(bits1), st()))

    conv1_packed()
    rows.append(Row(3, "conv1_forward_packed", "conv2d_relu forward, conv1, alive flags packed one bit per output",
                    conv1_packed, lambda: [y1p, bits1], conv1_flops, nbytes=conv1_bytes, bound="hbm",
                    cpu=lambda ref, w, r, bud: (lambda f, b: (f[0], [f[1], None]))(*conv_cpu(1, ref, w, r, bud)),
                    est_ms=0.006))
    y1q, bits1q, x2q = torch.empty_like(y1), torch.empty_like(bits1), torch.empty_like(x2)
    amax1 = torch.empty(N * 32 * 14 * 4, dtype=torch.uint8, device=dev)

    def conv1_pool1_packed():
        nnh.check(L.nnh_conv2d_relu_maxpool2d_forward_packed(P(dxc), N, 1, 28, 28, P(dw1), 32, 3, 3, P(db1), 1, 1,
                                                             P(y1q), P(bits1q), P(x2q), P(amax1), st()))

    conv1_pool1_packed()
    rows.append(Row(3, "conv1_pool1_forward_packed", "conv1 and the 2x2 s2 maxpool in one pass, alive flags as bits "
                    "and the window maxima as 2-bit positions", conv1_pool1_packed, lambda: [y1q, bits1q, x2q, amax1],
                    conv1_flops, nbytes=conv1_bytes + 4 * hx2.size, bound="hbm", est_ms=0.006))
    gx1p, gw1p, gb1p = torch.empty_like(dxc), torch.empty_like(dw1), torch.empty_like(db1)

    def conv1_bwd_packed():
        nnh.check(L.nnh_conv2d_backward_packed(P(g1), P(dxc), P(dw1), P(bits1), N, 1, 28, 28, 32, 3, 3, 1, 1, P(gx1p), 1,
                                               P(gw1p), 1, P(gb1p), 1, st()))

    rows.append(Row(3, "conv1_backward_packed", "conv2d_relu backward, conv1, from the packed flags: dx, dW, db",
                    conv1_bwd_packed, lambda: [gx1p, gw1p, gb1p], 2 * conv1_flops, nbytes=conv1_bwd_bytes, bound="hbm",
                    cpu=lambda ref, w, r, bud: (lambda f, b: (b[0], list(b[1])))(*conv_cpu(1, ref, w, r, bud)),
                    est_ms=0.02))
    gxpp = torch.empty_like(y1)

    def pool1_bwd_packed():
        nnh.check(L.nnh_maxpool2d_backward_packed(P(gp), P(amax1), N, 32, 28, 28, P(gxpp), 1, st()))

    rows.append(Row(3, "pool1_backward_packed", "maxpool2d backward 2x2 s2 from the 2-bit window positions",
                    pool1_bwd_packed, lambda: [gxpp], 0, nbytes=pool_bytes, bound="hbm",
                    cpu=lambda ref, w, r, bud: (lambda f, b: (b[0], [b[1]]))(*pool_cpu(ref, w, r, bud)),
                    est_ms=0.006))
    conv2_flops = 2.0 * N * 64 * 196 * 288
    rows.append(Row(3, "conv2_forward", "conv2d_relu forward, conv2: x [128,32,14,14] -> y [128,64,14,14], 3x3 s1 p1",
                    conv2, lambda: [y2], conv2_flops, nbytes=4 * (hx2.size + w2.size + 64 + N * 64 * 196),
                    cpu=lambda ref, w, r, bud: (lambda f, b: (f[0], [f[1]]))(*conv_cpu(2, ref, w, r, bud)),
                    f64=conv_fwd_f64(hx2, w2, b2, 289), est_ms=0.02))
    rows.append(Row(3, "conv2_backward", "conv2d_relu backward, conv2: dx, dW, db (g masked by alive)",
                    conv_bwd(g2, x2, dw2, al2, (N, 32, 14, 14), (gx2, gw2, gb2)), lambda: [gx2, gw2, gb2],
                    2 * conv2_flops,
                    cpu=lambda ref, w, r, bud: (lambda f, b: (b[0], list(b[1])))(*conv_cpu(2, ref, w, r, bud)),
                    f64=conv_bwd_f64(hg2, hy2, hx2, w2, 196), est_ms=0.05))

    # config 4: attention, batch 32, 8 heads, seq 256, head width 64 (+ causal); probs stored, as the reference does
    Na, T, D, H = 32, 256, 512, 8
    q, k, v = (synth.normal(3 + i, (Na, T, D)) for i in range(3))
    hg = synth.normal(7, (Na, T, D))
    dq_, dk_, dv_, ga = d(q), d(k), d(v), d(hg)
    att_flops = 2 * 2.0 * Na * H * T * T * (D // H)
    useful = 2 * 2.0 * Na * H * (T * (T + 1) // 2) * (D // H)
    att_cache = {}

    def att_cpu(causal, ref, w, r, bud):
        if (causal, w, r, bud) not in att_cache:
            att_cache[(causal, w, r, bud)] = ref.time_attention(q, k, v, H, causal, hg, w, r, bud)
        return att_cache[(causal, w, r, bud)]

    f64_cache = {}

    def att_f64(causal):
        if causal not in f64_cache:
            f64_cache[causal] = _attention_f64(q, k, v, hg, H, causal)
        return f64_cache[causal]

    for causal in (False, True):
        out = torch.empty((Na, T, D), device=dev)
        probs = torch.empty((Na, H, T, T), device=dev)
        gq, gk, gv = torch.empty_like(dq_), torch.empty_like(dk_), torch.empty_like(dv_)

        def fwd(out=out, probs=probs, causal=causal):
            nnh.check(L.nnh_attention_forward(P(dq_), P(dk_), P(dv_), Na, T, T, D, H, None, causal, P(out), P(probs),
                                              st()))

        def bwd(probs=probs, gq=gq, gk=gk, gv=gv, causal=causal):
            nnh.check(L.nnh_attention_backward(P(ga), P(dq_), P(dk_), P(dv_), P(probs), Na, T, T, D, H, None, causal,
                                               P(gq), 1, P(gk), 1, P(gv), 1, st()))

        fwd()
        tag = " causal" if causal else ""
        rows.append(Row(4, "attention_forward" + ("_causal" if causal else ""),
                        f"nn::attention forward{tag}: q, k, v [32,256,512], 8 heads of 64, probs stored", fwd,
                        lambda out=out: [out], att_flops, useful_flops=useful if causal else None,
                        cpu=lambda ref, w, r, bud, c=causal: (lambda f, b: (f[0], [f[1]]))(*att_cpu(c, ref, w, r, bud)),
                        f64=lambda h, c=causal: _vs_f64(h[0], att_f64(c)[0]), est_ms=0.085))
        rows.append(Row(4, "attention_backward" + ("_causal" if causal else ""),
                        f"nn::attention backward{tag}: dQ, dK, dV", bwd, lambda gq=gq, gk=gk, gv=gv: [gq, gk, gv],
                        2 * att_flops, useful_flops=2 * useful if causal else None,
                        cpu=lambda ref, w, r, bud, c=causal: (lambda f, b: (b[0], list(b[1])))(*att_cpu(c, ref, w, r, bud)),
                        f64=lambda h, c=causal: _worst([_vs_f64(g_, w_) for g_, w_ in zip(h, att_f64(c)[1])]),
                        est_ms=0.13))

    # config 5: the roofline sweep through nn::matmul (seed 4)
    for (m5, n5, k5, est) in ((1024, 1024, 1024, 0.027), (2048, 2048, 2048, 0.16), (4096, 4096, 4096, 1.15),
                              (8192, 8192, 8192, 9.1), (64, 4096, 4096, 0.06), (4096, 4096, 64, 0.028)):
        matmul_row(5, f"matmul_{m5}x{n5}x{k5}", f"nn::matmul {m5}x{n5}x{k5} C = A B", 4, m5, n5, k5, 0, 0, est)
    return rows


def build_next_rows():
    """The memory-bound ops next to the path on nn-cpp's own workloads (not BASELINE configs): batchnorm with its
    folded ReLU at cnn_fer's first Conv-BN-ReLU (x [64,16,48,48], apps/bench/workloads.cpp:185-199) and layernorm
    over config 4's activations (x [32,256,512]) and transformer_tiny's ([16,64,64]), forward and backward. Inputs
    are seeded U[-3,5] activations, U[0.5,1.5] scales, U[-1,1] shifts and N(0,1) output gradients; HBM-bound, the
    algorithmic bytes count x (and g) read once and y (dx) written once, not the alive flags or the per-channel or
    per-row statistics."""
    import numpy as np
    import torch

    import nnh
    from nnh import synth
    L = nnh.lib()
    dev = torch.device("cuda:0")
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    st = lambda: nnh._stream(None)
    P = nnh._ptr
    rows = []
    # batchnorm + ReLU, cnn_fer layer 1
    N, Cc, H, W = 64, 16, 48, 48
    S = H * W
    hx = (synth.mt19937_uniform(41, N * Cc * S, -3.0, 5.0)).reshape(N, Cc, H, W)
    hw = synth.mt19937_uniform(42, Cc, 0.5, 1.5)
    hb = synth.mt19937_uniform(43, Cc, -1.0, 1.0)
    hg = synth.normal(44, (N, Cc, H, W))
    x, w, b, g = d(hx), d(hw), d(hb), d(hg)
    y, dx = torch.empty_like(x), torch.empty_like(x)
    alive = torch.empty(x.shape, dtype=torch.uint8, device=dev)
    mean, var, inv = (torch.empty(Cc, device=dev) for _ in range(3))
    dw, db = torch.empty(Cc, device=dev), torch.empty(Cc, device=dev)

    def bn_fwd():
        nnh.check(L.nnh_batchnorm_forward(P(x), N, Cc, S, P(w), P(b), 1e-5, 1, P(y), P(alive), P(mean), P(var), P(inv),
                                          st()))

    def bn_bwd():
        nnh.check(L.nnh_batchnorm_backward(P(g), P(x), P(alive), P(w), P(mean), P(inv), N, Cc, S, P(dx), 1, P(dw), 1,
                                           P(db), 1, st()))

    bn_fwd()
    bn_cache = {}

    def bn_cpu(ref, wu, r, bud):
        if (wu, r, bud) not in bn_cache:
            bn_cache[(wu, r, bud)] = ref.time_batchnorm(hx, hw, hb, 1e-5, 1, hg, wu, r, bud)
        return bn_cache[(wu, r, bud)]

    xb = 4 * hx.size
    rows.append(Row("next", "batchnorm_relu_forward", "nn::batchnorm + folded ReLU forward, cnn_fer layer 1: "
                    "x [64,16,48,48] (training-mode batch statistics)", bn_fwd, lambda: [y], 0, nbytes=2 * xb,
                    bound="hbm", cpu=lambda ref, wu, r, bud: (lambda f, bw: (f[0], [f[1]]))(*bn_cpu(ref, wu, r, bud)),
                    est_ms=0.02))
    rows.append(Row("next", "batchnorm_relu_backward", "nn::batchnorm + folded ReLU backward: dx, dweight, dbias",
                    bn_bwd, lambda: [dx, dw, db], 0, nbytes=3 * xb, bound="hbm",
                    cpu=lambda ref, wu, r, bud: (lambda f, bw: (bw[0], [bw[1], None, None]))(*bn_cpu(ref, wu, r, bud)),
                    est_ms=0.02))
    for key, shape, seed in (("layernorm_attention_acts", (32, 256, 512), 45), ("layernorm_transformer_tiny",
                                                                               (16, 64, 64), 46)):
        D = shape[-1]
        R = int(np.prod(shape)) // D
        hlx = synth.mt19937_uniform(seed, R * D, -3.0, 5.0).reshape(shape)
        hgm = synth.mt19937_uniform(seed + 10, D, 0.5, 1.5)
        hbt = synth.mt19937_uniform(seed + 20, D, -1.0, 1.0)
        hlg = synth.normal(seed + 30, shape)
        lx, gm, bt, lg = d(hlx), d(hgm), d(hbt), d(hlg)
        ly, ldx = torch.empty_like(lx), torch.empty_like(lx)
        lmean, linv = torch.empty(R, device=dev), torch.empty(R, device=dev)
        dgm, dbt = torch.empty(D, device=dev), torch.empty(D, device=dev)

        def ln_fwd(lx=lx, gm=gm, bt=bt, ly=ly, lmean=lmean, linv=linv, R=R, D=D):
            nnh.check(L.nnh_layernorm_forward(P(lx), R, D, P(gm), P(bt), 1e-5, P(ly), P(lmean), P(linv), st()))

        def ln_bwd(lg=lg, lx=lx, gm=gm, lmean=lmean, linv=linv, ldx=ldx, dgm=dgm, dbt=dbt, R=R, D=D):
            nnh.check(L.nnh_layernorm_backward(P(lg), P(lx), P(gm), P(lmean), P(linv), R, D, P(ldx), 1, P(dgm), 1,
                                               P(dbt), 1, st()))

        ln_fwd()
        cache = {}

        def ln_cpu(ref, wu, r, bud, hlx=hlx, hgm=hgm, hbt=hbt, hlg=hlg, cache=cache):
            if (wu, r, bud) not in cache:
                cache[(wu, r, bud)] = ref.time_layernorm(hlx, hgm, hbt, 1e-5, hlg, wu, r, bud)
            return cache[(wu, r, bud)]

        lb = 4 * hlx.size
        dims = "x".join(map(str, shape))
        rows.append(Row("next", key + "_forward", f"nn::layernorm forward over the last axis of [{dims}]", ln_fwd,
                        lambda ly=ly: [ly], 0, nbytes=2 * lb, bound="hbm",
                        cpu=lambda ref, wu, r, bud, f=ln_cpu: (lambda a, bw: (a[0], [a[1]]))(*f(ref, wu, r, bud)),
                        est_ms=0.02))
        rows.append(Row("next", key + "_backward", f"nn::layernorm backward over [{dims}]: dx, dgamma, dbeta", ln_bwd,
                        lambda ldx=ldx, dgm=dgm, dbt=dbt: [ldx, dgm, dbt], 0, nbytes=3 * lb, bound="hbm",
                        cpu=lambda ref, wu, r, bud, f=ln_cpu: (lambda a, bw: (bw[0], [bw[1], None, None]))(
                            *f(ref, wu, r, bud)),
                        est_ms=0.03))
    return rows


def run_gpu_rows(rows):
    """Times every row on the GPU, checks that three runs give the same bits, and keeps one run's outputs on the
    host."""
    import torch
    for r in rows:
        times = device_times(r.gpu, r.est_ms)
        ms = median(times)
        res = {"ms": ms, "spread": spread(times), "runs": len(times)}
        outs = []
        for rep in range(3):
            r.gpu()
            torch.cuda.synchronize()
            cur = [t.clone() for t in r.outs()]
            outs.append(cur)
        same = all(torch.equal(a.view(torch.int32), b.view(torch.int32)) for a, b in zip(outs[0], outs[1])) and \
            all(torch.equal(a.view(torch.int32), b.view(torch.int32)) for a, b in zip(outs[0], outs[2]))
        res["bitwise_repeat"] = bool(same)
        r.host_outs = [t.cpu().numpy() for t in outs[0]]
        del outs
        if r.flops:
            res["tflops"] = r.flops / (ms * 1e-3) / 1e12
        if r.nbytes:
            res["gbps"] = r.nbytes / (ms * 1e-3) / 1e9
        achieved = res["tflops"] if r.bound == "mfma" else res["gbps"]
        peak = PEAK_FP32_MFMA_TFLOPS if r.bound == "mfma" else PEAK_HBM_GBPS
        res["roofline"] = {"bound": r.bound, "achieved": achieved, "peak": peak,
                           "unit": "TFLOP/s" if r.bound == "mfma" else "GB/s", "frac": achieved / peak}
        if r.useful_flops:
            res["roofline"]["useful_frac"] = r.useful_flops / (ms * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS
        r.result = res
        log(f"[cfg {r.cfg}] {r.key}: {ms * 1e3:.2f} us (spread {res['spread']:.3f}), "
            f"{achieved:.1f} {res['roofline']['unit']} = {res['roofline']['frac'] * 100:.1f}% of {r.bound} peak, "
            f"repeat bitwise {same}")


def unpack_argmax2(a2, planes, h, w):
    """The plane offsets of nnh.h's 2-bit window positions (2 x 2, stride 2): {planes, h / 2, w / 2} uint32."""
    import numpy as np
    ph, pw, rb = h // 2, w // 2, (w + 7) // 8
    j = np.arange(pw)
    slot = (a2.reshape(planes, ph, rb)[:, :, j // 4] >> (2 * (j % 4)).astype(np.uint8)) & 3
    rows = 2 * np.arange(ph)[None, :, None] + slot // 2
    return (rows * w + 2 * j[None, None, :] + slot % 2).astype(np.uint32)


def packed_checks(by_key):
    """Each packed row against its byte-form row, bit for bit: values and gradients equal, flags equal to the
    bytes' np.packbits (little bit order), window positions decoding to the 32-bit offsets."""
    import numpy as np
    eq = lambda a, b: a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))
    fused = by_key.get("conv1_pool1_forward")
    pairs = {"conv1_forward_packed": "conv1_forward", "conv1_pool1_forward_packed": "conv1_pool1_forward",
             "conv1_backward_packed": "conv1_backward", "pool1_backward_packed": "pool1_backward"}
    for key, base in pairs.items():
        r, b = by_key.get(key), by_key.get(base)
        if r is None or b is None:
            continue
        h, w = r.host_outs, b.host_outs
        if key == "conv1_forward_packed":
            ok = eq(h[0], w[0]) and fused is not None and \
                eq(h[1], np.packbits(fused.host_outs[1].reshape(-1), bitorder="little"))
        elif key == "conv1_pool1_forward_packed":
            ok = eq(h[0], w[0]) and eq(h[2], w[2]) and \
                eq(h[1], np.packbits(w[1].reshape(-1), bitorder="little")) and \
                eq(unpack_argmax2(h[3], 128 * 32, 28, 28).reshape(-1), w[3].view(np.uint32).reshape(-1))
        else:
            ok = len(h) == len(w) and all(eq(x, y) for x, y in zip(h, w))
        r.result["bitwise_vs_byte_form"] = bool(ok)


def run_cpu_rows(rows, headline=None):
    """nn-cpp's own op on the same host buffers for every row with a CPU counterpart: one thread per physical core
    (pinned) and one thread; the last run's outputs are compared with the GPU's. Returns the baseline's setup."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from pyoracle import Reference, reference_available
    if not reference_available():
        log("cpu baseline: oracle/_ref not built; skipped")
        return None
    cores, allowed = physical_cores()
    saved = os.sched_getaffinity(0)
    ref = Reference()
    setup = {"cpu": cpu_model(), "governor": cpu_governor(), "allowed_cpus": allowed, "physical_cores": len(cores),
             "pinned_to": cores, "build": "nn-cpp 2.0.0 NN_NATIVE (g++ -O3 -mavx2 -mfma -ffp-contract=off)"}
    log(f"cpu baseline: {setup['cpu']}, governor {setup['governor']}, {len(cores)} physical cores of {allowed} "
        f"allowed CPUs")
    try:
        for threads, budget, max_runs, key in ((len(cores), 1.5, 15, "cpu_baseline"), (1, 1.0, 5, "cpu_1thread")):
            os.sched_setaffinity(0, cores[:threads])
            ref.set_threads(threads)
            for r in rows + ([headline] if headline is not None and threads == len(cores) else []):
                if r.cpu is None:
                    continue
                t0 = time.perf_counter()
                # one untimed call first (page faults, the pool's start); a single run past the budget counts as it
                times, outs = r.cpu(ref, 0, 1, 0.0)
                warm = times[0] * 1e-3 < budget
                if warm:
                    times, outs = r.cpu(ref, 0, max_runs, budget)
                ms = median(times)
                entry = {"ms": ms, "spread": spread(times), "runs": len(times), "threads": threads,
                         "warmup": 1 if warm else 0}
                if r.flops:
                    entry["tflops"] = r.flops / (ms * 1e-3) / 1e12
                if key == "cpu_baseline" and hasattr(r, "host_outs"):
                    pairs = [(g, w) for g, w in zip(r.host_outs, outs) if w is not None]
                    same = all(np.array_equal(g.view(np.uint32), w.reshape(g.shape).view(np.uint32)) for g, w in pairs)
                    diff = max(float(np.max(np.abs(g.astype(np.float64) - w.reshape(g.shape).astype(np.float64))))
                               if g.size else 0.0 for g, w in pairs)
                    r.result["bitwise_vs_nn_cpp"] = bool(same)
                    r.result["maxabs_vs_nn_cpp"] = diff
                r.result[key] = entry
                log(f"  [{key} x{threads}] {r.key}: {ms:.3f} ms median of {len(times)} "
                    f"({time.perf_counter() - t0:.1f} s)")
    finally:
        os.sched_setaffinity(0, saved)
    return setup


def run_workloads(with_cpu=True, seed=1, warmup=3, runs=15):
    """nn-cpp's bench models (apps/bench/workloads.cpp:80-137; the definitions are nnh/workloads.py): parameters
    reseeded from std::mt19937(seed) and the input drawn from std::mt19937(seed + 1), as make_workload does; one
    training step's forward pass and its zero_grad plus backward pass (from a fixed N(0,1) gradient of the logits; no
    loss, no optimizer step), timed as runner.cpp:33-45 does, median of `runs` after `warmup`: on the GPU through
    nn::hip (libnnh_workloads.so), and nn-cpp's own step on the CPU (one thread per physical core, pinned), the logits
    compared bit for bit."""
    import ctypes as C

    import numpy as np

    from nnh import workloads as wl
    L = C.CDLL(os.path.join(ROOT, "nn-cpp_amd", "lib", "libnnh_workloads.so"))
    ref = None
    if with_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        from pyoracle import Reference, reference_available
        if reference_available():
            ref = Reference()
    out = []
    for w in wl.WORKLOADS:
        params, x, g = wl.inputs(w, seed)
        res = {"workload": w.name, "batch": w.batch}
        for side, lib, fn in (("gpu", L, "nnh_bench_workload_step"), ("cpu", ref.lib if ref else None,
                                                                       "nnref_time_workload_step")):
            if lib is None:
                continue
            if side == "cpu":
                cores, _ = physical_cores()
                saved = os.sched_getaffinity(0)
                os.sched_setaffinity(0, cores)
                ref.set_threads(len(cores))
            try:
                rc, fwd, bwd, logits, _ = wl.run_step(getattr(lib, fn), w, params, x, g, warmup, runs)
            finally:
                if side == "cpu":
                    os.sched_setaffinity(0, saved)
            assert rc == 0, (w.name, side, rc)
            tot = list(fwd + bwd)
            res[side] = {"forward_ms": median(list(fwd)), "backward_ms": median(list(bwd)), "total_ms": median(tot),
                         "spread": spread(tot), "runs": runs}
            if side == "cpu":
                res["cpu"]["threads"] = len(physical_cores()[0])
            res[side + "_logits"] = logits
        if "cpu" in res:
            res["bitwise_vs_nn_cpp"] = bool(np.array_equal(res["gpu_logits"].view(np.uint32),
                                                           res["cpu_logits"].view(np.uint32)))
            res["speedup_gpu"] = res["cpu"]["total_ms"] / res["gpu"]["total_ms"]
        for k in ("gpu_logits", "cpu_logits"):
            res.pop(k, None)
        log(f"[workload] {w.name}: GPU forward {res['gpu']['forward_ms']:.3f} ms + backward "
            f"{res['gpu']['backward_ms']:.3f} ms" + (f"; nn-cpp CPU {res['cpu']['total_ms']:.3f} ms; logits bitwise "
                                                     f"{res['bitwise_vs_nn_cpp']}" if "cpu" in res else ""))
        out.append(res)
    return out


def csv_size(key, cfg):
    """The CSV's size column: run_matmul's n for the square products (runner.cpp:80-96), m x n x k for the other
    config-5 products, the config number for the op rows."""
    m = re.match(r"matmul(\d+)_[nt][nt]$", key)
    if m:
        return m.group(1)
    if key.startswith("matmul_"):
        return key[len("matmul_"):]
    return str(cfg)


def write_csv(path, rows, setup, workloads=()):
    """apps/bench/bench.cpp:112-113's columns, then the GPU columns; one line per GPU row and per CPU baseline."""
    cols = ["config", "label", "threads", "benchmark", "size", "forward_ms", "backward_ms", "optim_ms", "total_ms",
            "gflops", "spread", "runs", "tflops", "gbps", "roofline_bound", "roofline_frac", "maxabs_err",
            "bitwise_repeat"]
    lines = [",".join(cols)]
    f = lambda v: "" if v is None else (f"{v:.6g}" if isinstance(v, float) else str(v))
    for r in rows:
        res = r.result
        back = "backward" in r.key
        size = csv_size(r.key, r.cfg)
        for label, ent, thr in (("gpu-mi355x", res, ""), ("native-pinned", res.get("cpu_baseline"), None),
                                ("native-1thread", res.get("cpu_1thread"), None)):
            if not ent:
                continue
            ms = ent["ms"]
            gpu = label.startswith("gpu")
            vals = ["gpu" if gpu else "native", label, thr if gpu else ent["threads"], r.key, size,
                    None if back else ms, ms if back else None, None, ms,
                    r.flops / (ms * 1e6) if r.flops else None, ent["spread"], ent["runs"],
                    res.get("tflops") if gpu else ent.get("tflops"), res.get("gbps") if gpu else None,
                    r.bound if gpu else None, res["roofline"]["frac"] if gpu else None,
                    res.get("maxabs_vs_nn_cpp") if gpu else None, res.get("bitwise_repeat") if gpu else None]
            lines.append(",".join(f(v) for v in vals))
    for w in workloads:
        for side, label in (("gpu", "gpu-mi355x"), ("cpu", "native-pinned")):
            if side not in w:
                continue
            e = w[side]
            vals = ["gpu" if side == "gpu" else "native", label, "" if side == "gpu" else e["threads"], w["workload"],
                    str(w["batch"]), e["forward_ms"], e["backward_ms"], None, e["total_ms"], None, e["spread"],
                    e["runs"], None, None, None, None, None, None]
            lines.append(",".join(f(v) for v in vals))
    with open(path, "w") as fh:
        fh.write("\n".join(lines) + "\n")
    log(f"csv: {path} ({len(lines) - 1} rows)")


def row_json(r):
    res = r.result
    out = {"cfg": r.cfg, "key": r.key, "workload": r.workload, "ms": round(res["ms"], 6),
           "spread": round(res["spread"], 4), "runs": res["runs"]}
    for k in ("tflops", "gbps"):
        if k in res:
            out[k] = round(res[k], 3)
    out["roofline"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in res["roofline"].items()}
    for k in ("bitwise_repeat", "bitwise_vs_nn_cpp", "bitwise_vs_two_ops", "bitwise_vs_byte_form"):
        if k in res:
            out[k] = res[k]
    if "maxabs_vs_nn_cpp" in res and not res.get("bitwise_vs_nn_cpp", True):
        out["maxabs_vs_nn_cpp"] = res["maxabs_vs_nn_cpp"]
    for k in ("cpu_baseline", "cpu_1thread"):
        if k in res:
            e = res[k]
            out[k] = {"ms": round(e["ms"], 4), "threads": e["threads"], "runs": e["runs"],
                      "spread": round(e["spread"], 4), "speedup_gpu": round(e["ms"] / res["ms"], 1)}
    return out


LINE_LIMIT = 4096  # bytes: the stdout line the driver parses stays well inside what it keeps of stdout


def _r(v, nd):
    return None if v is None else round(v, nd)


def compact_row(row):
    """One config row as the stdout line carries it (under its key): median device ms, roofline fraction, nn-cpp's pinned CPU
    ms, and whether the outputs were the same bits over three GPU runs and against nn-cpp (against the exact mode's
    outputs' bits are not asked of a split-depth row: there `bitwise` is the repeat check alone)."""
    bits = row.get("bitwise_repeat", False) and row.get("bitwise_vs_nn_cpp", True)
    if row["key"].endswith("_split"):
        bits = row.get("bitwise_repeat", False)
    out = {"ms": _r(row["ms"], 5), "frac": _r(row["roofline"]["frac"], 4), "bitwise": bool(bits)}
    if not row["key"].endswith("_split"):
        out["cpu_ms"] = _r((row.get("cpu_baseline") or {}).get("ms"), 3)
    if "useful_frac" in row["roofline"]:
        out["useful_frac"] = _r(row["roofline"]["useful_frac"], 4)
    return out


def compact_line(full, strict=True):
    """The driver's JSON line from the full result: the headline keys, roofline and cpu_baseline, the fused-op
    figure, and per row only compact_row's fields; the full rows go to a file and to stderr. Past LINE_LIMIT it
    raises when strict, else first sheds the workloads, the split-depth rows and the fused-op object."""
    keep = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "settle_launches", "ms_per_step",
            "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline")
    line = {k: full.get(k) for k in keep}
    line["data"] = DATA_SHORT
    fo = full.get("fused_op")
    if fo:
        line["fused_op"] = {"workload": "conv1 fwd + alive (cfg 3)", "value": fo["value"],
                            "unit": fo["unit"], "us": fo["us_per_launch"], "frac": fo["roofline"]["frac"],
                            "frac_of_fill_floor": (fo.get("fill_floor") or {}).get("conv1_frac_of_floor")}
        # the packed-flag rows: their times and whether all four gave the byte forms' bits (full rows: the rest)
        packed = {r["key"]: r for r in full.get("configs", []) if r["key"].endswith("_packed")}
        if packed:
            short = {"conv1_forward_packed": "fwd", "conv1_pool1_forward_packed": "fwd_pool",
                     "conv1_backward_packed": "bwd", "pool1_backward_packed": "pool_bwd"}
            line["fused_op"]["packed_us"] = {short.get(k, k): _r(r["ms"] * 1e3, 2) for k, r in packed.items()}
            line["fused_op"]["packed_us"]["bitwise"] = all(r.get("bitwise_vs_byte_form") is True and
                                                           r.get("bitwise_repeat", False) for r in packed.values())
    line["configs"] = {r["key"]: compact_row(r) for r in full.get("configs", []) if not r["key"].endswith("_packed")}
    line["configs_split_depth"] = {r["key"]: compact_row(r) for r in full.get("configs_split_depth", [])}
    line["workloads"] = [{"workload": w["workload"], "gpu_ms": _r(w.get("gpu", {}).get("total_ms"), 4),
                          "cpu_ms": _r((w.get("cpu") or {}).get("total_ms"), 4),
                          "bitwise": w.get("bitwise_vs_nn_cpp")} for w in full.get("workloads", [])]
    if line["workloads"]:
        line["workloads_note"] = WORKLOAD_NOTE_SHORT
    line["full_rows"] = full.get("full_rows")
    text = json.dumps(line, separators=(",", ":"))
    if len(text.encode()) > LINE_LIMIT and not strict:
        # never lose the line: shed what the full rows also hold, least important first
        for drop in ("workloads_note", "workloads", "configs_split_depth", "fused_op"):
            line.pop(drop, None)
            text = json.dumps(line, separators=(",", ":"))
            if len(text.encode()) <= LINE_LIMIT:
                break
    if len(text.encode()) > LINE_LIMIT:
        raise ValueError(f"bench line is {len(text.encode())} bytes, over {LINE_LIMIT}")
    return text


DATA_SHORT = "synthetic: nn-cpp's seeded mt19937 streams (N(0,1): numpy PCG64); same buffers both sides"
WORKLOAD_NOTE = ("step = forward + zero_grad + backward from a fixed N(0,1) logits gradient, both sides; no loss, "
                 "no optimizer step (runner.cpp's optim_ms)")
WORKLOAD_NOTE_SHORT = "step = fwd + zero_grad + bwd from fixed N(0,1) logits grads; no loss, no optimizer step"


def report(with_cpu=True):
    """The config rows as a markdown table, with the fp64 checks (slow)."""
    import torch
    rows = build_rows(report=True) + build_next_rows()
    run_gpu_rows(rows)
    setup = run_cpu_rows(rows) if with_cpu else None
    for r in rows:
        if r.f64:
            r.result["f64"] = r.f64(r.host_outs)
    lines = [f"GPU: {torch.cuda.get_device_name(0)}; nn-cpp CPU baseline: " +
             (f"{setup['build']}, {setup['physical_cores']} threads pinned one per physical core of {setup['cpu']} "
              f"(governor {setup['governor']}), and 1 thread" if setup else "not run"), "",
             "| cfg | workload | GPU ms (median) | spread | TFLOP/s | GB/s | bound | % of roofline | nn-cpp CPU ms | "
             "nn-cpp 1-thread ms | GPU speedup | 3 GPU runs | vs nn-cpp | max abs err vs fp64 | err / bound |",
             "|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    f = lambda v, fmt: (fmt % v) if v is not None else "-"
    for r in rows:
        res = r.result
        cb, c1 = res.get("cpu_baseline"), res.get("cpu_1thread")
        fe = res.get("f64") or (None, None)
        vs = "-" if "bitwise_vs_nn_cpp" not in res else ("0 (bitwise)" if res["bitwise_vs_nn_cpp"]
                                                         else "%.3g" % res["maxabs_vs_nn_cpp"])
        lines.append(f"| {r.cfg} | {r.workload} | {res['ms']:.4f} | {res['spread']:.3f} | {f(res.get('tflops'), '%.2f')} | "
                     f"{f(res.get('gbps'), '%.0f')} | {r.bound} | {res['roofline']['frac'] * 100:.1f}% | "
                     f"{f(cb['ms'] if cb else None, '%.3f')} | {f(c1['ms'] if c1 else None, '%.3f')} | "
                     f"{f(cb['ms'] / res['ms'] if cb else None, '%.0fx')} | "
                     f"{'bitwise equal' if res['bitwise_repeat'] else 'DIFFER'} | {vs} | {f(fe[0], '%.3g')} | "
                     f"{f(fe[1], '%.3g')} |")
    print("\n".join(lines), flush=True)


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


def make_parser():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--size", type=int, default=4096)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="only the headline product (no per-config rows)")
    ap.add_argument("--no-split", action="store_true", help="no rows in the split-depth numerics mode")
    ap.add_argument("--csv", default=None, help="also write the rows as CSV (the reference's bench columns + GPU ones)")
    ap.add_argument("--full-json", default=os.path.join("gpurun_out", "bench_full.json"), metavar="PATH",
                    help="where the full rows (every field, split-depth, next rows, workloads) are written; the "
                         "stdout line carries a compact form")
    ap.add_argument("--report", action="store_true", help="every BASELINE config as a markdown table with fp64 "
                    "checks (not the driver's JSON line)")
    ap.add_argument("--row", default=None, metavar="KEY", help="time one configuration row only (its key, e.g. "
                    "conv1_forward, or matmul512_nt_split in the split-depth mode) and print its JSON: the command "
                    "the per-kernel profiles under profiles/ are taken with")
    ap.add_argument("--workloads", action="store_true", help="only nn-cpp's bench models' training steps (GPU and "
                    "nn-cpp CPU), one JSON line")
    ap.add_argument("--floor", action="store_true", help="launch-cost floor of this GPU: empty kernel, fills, copies")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run 5 device-to-device copies of MIB MiB (calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return ap


def main():
    args = make_parser().parse_args()
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
    if args.workloads:
        import torch  # noqa: F401 (torch's HIP runtime first, as everywhere else)
        res = run_workloads(with_cpu=not args.no_cpu_baseline)
        print(json.dumps({"workloads": [{k: ({kk: (round(vv, 4) if isinstance(vv, float) else vv)
                                                for kk, vv in v.items()} if isinstance(v, dict) else v)
                                           for k, v in w.items()} for w in res]}), flush=True)
        return
    if args.row:
        import torch  # noqa: F401 (torch's HIP runtime first, as everywhere else; libnnh then shares it)

        import nnh
        split = args.row.endswith("_split")
        prev = nnh.set_numerics(nnh.NUMERICS_SPLIT_DEPTH if split else nnh.NUMERICS_NNCPP)
        try:
            rows = build_rows(split=split) + ([] if split else build_next_rows())
            keys = [r.key for r in rows]
            rows = [r for r in rows if r.key == args.row]
            if not rows:
                print(f"bench.py: no row {args.row!r}; rows: {', '.join(keys)}", file=sys.stderr)
                sys.exit(2)
            run_gpu_rows(rows)
        finally:
            nnh.set_numerics(prev)
        print(json.dumps(row_json(rows[0])), flush=True)
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

    # settle the clock, then the driver's warm-up steps, then exactly K timed steps between two synchronisations
    settle = 0
    t_end = time.perf_counter() + SETTLE_S
    while settle < 20 or time.perf_counter() < t_end:
        step()
        settle += 1
        if settle % 20 == 0:
            torch.cuda.synchronize()
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
        f"{value:.2f} TFLOP/s wall over {args.steps} steps after {settle} settling launches")
    del dc

    rows = []
    fill_floor_ms = None
    if not args.no_configs:
        rows = build_rows()
        run_gpu_rows(rows)
        by_key = {r.key: r for r in rows}
        fused = by_key.get("conv1_pool1_forward")
        if fused is not None and "conv1_forward" in by_key and "pool1_forward" in by_key:
            want = by_key["conv1_forward"].host_outs[:1] + [None] + by_key["pool1_forward"].host_outs
            fused.result["bitwise_vs_two_ops"] = all(w is None or np.array_equal(g.view(np.uint8), w.view(np.uint8))
                                                     for g, w in zip(fused.host_outs, want))
        packed_checks(by_key)
        # the launch floor of conv1's output size on this GPU: a plain fill of y (12.85 MB)
        ny = 128 * 32 * 28 * 28
        fill_buf = torch.empty(ny, device=dev)
        fill_floor_ms = median(device_times(lambda: fill_buf.fill_(1.0), 0.004))
        del fill_buf
    split_rows = []
    if not args.no_configs and not args.no_split:
        prev = nnh.set_numerics(nnh.NUMERICS_SPLIT_DEPTH)
        try:
            split_rows = build_rows(split=True)
            run_gpu_rows(split_rows)
        finally:
            nnh.set_numerics(prev)
        exact = {r.key: r for r in rows}
        for r in split_rows:
            e = exact.get(r.key[: -len("_split")])
            if e is not None:
                r.result["bitwise_vs_nn_cpp"] = all(np.array_equal(g.view(np.uint32), w.view(np.uint32))
                                                    for g, w in zip(r.host_outs, e.host_outs))
                r.result["maxabs_vs_nn_cpp"] = max(float(np.max(np.abs(g.astype(np.float64) - w)))
                                                   for g, w in zip(r.host_outs, e.host_outs))
    next_rows = []
    if not args.no_configs:
        next_rows = build_next_rows()
        run_gpu_rows(next_rows)
    headline = Row(5, "headline", f"nn::kernels::sgemm {m}^3", None, None, flops,
                   cpu=lambda ref, w, r, bud: ref.time_matmul(a, b, 0, 0, w, r, bud))
    setup = None
    if not args.no_cpu_baseline:
        setup = run_cpu_rows(rows + next_rows, headline)
    workloads = [] if args.no_configs else run_workloads(with_cpu=not args.no_cpu_baseline)
    if args.csv and rows:
        write_csv(args.csv, rows + next_rows, setup, workloads)
    cpu = None
    hb = headline.result.get("cpu_baseline")
    if hb:
        cpu = {"value": round(flops / (hb["ms"] * 1e-3) / 1e12, 4), "unit": "TFLOP/s", "cores": hb["threads"],
               "kind": "reference",
               "sample": (f"nn::matmul {m}^3, nn-cpp NN_NATIVE AVX2 build (oracle/_ref), same seed-4 inputs, "
                          f"{hb['threads']} threads pinned 1/physical core of {setup['cpu']} ({setup['governor']}), "
                          f"median of {hb['runs']} after {hb['warmup']} warm-up")}
    conv1 = next((r for r in rows if r.key == "conv1_forward"), None)
    conv1_na = next((r for r in rows if r.key == "conv1_forward_no_alive"), None)
    pool1 = next((r for r in rows if r.key == "pool1_forward"), None)
    conv1_pool1 = next((r for r in rows if r.key == "conv1_pool1_forward"), None)
    fill_gbps = None if fill_floor_ms is None else 4 * 128 * 32 * 784 / (fill_floor_ms * 1e-3) / 1e9
    out = {
        "metric": "fp32 GEMM TFLOP/s @4096^3 + % MI355X fp32 MFMA peak; fused-op GB/s",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_launches": settle,
        "ms_per_step": round(wall / args.steps * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: the reference's seeded streams (std::mt19937(seed) + uniform_real_distribution<float>; "
                "N(0,1) from numpy's PCG64 where BASELINE.json asks for normal values); both sides get the same buffers",
        "config": {"workload": f"sgemm {m}x{n}x{k} NN fp32 (BASELINE config 5)", "m": m, "n": n, "k": k,
                   "trans_a": False, "trans_b": False, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_FP32_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4),
                     "traffic": traffic_from_profile(f"sgemm_{m}")},
        "cpu_baseline": cpu,
        "cpu_setup": setup,
        "fused_op": None if conv1 is None else {
            "workload": conv1.workload, "value": round(conv1.result["gbps"], 1), "unit": "GB/s",
            "us_per_launch": round(conv1.result["ms"] * 1e3, 3), "algorithmic_bytes": conv1.nbytes,
            "roofline": {"bound": "hbm", "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                         "frac": round(conv1.result["roofline"]["frac"], 4)},
            "without_alive_flags": None if conv1_na is None else {
                "us_per_launch": round(conv1_na.result["ms"] * 1e3, 3), "value": round(conv1_na.result["gbps"], 1)},
            "fill_floor": None if fill_floor_ms is None else {
                "what": "torch fill of conv1's y (12.85 MB) on this GPU, the fastest a launch writing it runs",
                "us_per_launch": round(fill_floor_ms * 1e3, 3), "value": round(fill_gbps, 1),
                "frac_of_peak": round(fill_gbps / PEAK_HBM_GBPS, 4),
                "conv1_frac_of_floor": round(conv1.result["gbps"] / fill_gbps, 4)},
            "with_pool": None if conv1_pool1 is None or pool1 is None else {
                "workload": conv1_pool1.workload, "us_per_launch": round(conv1_pool1.result["ms"] * 1e3, 3),
                "separate_us": round((conv1.result["ms"] + pool1.result["ms"]) * 1e3, 3),
                "bitwise_vs_two_ops": conv1_pool1.result.get("bitwise_vs_two_ops")},
            "packed_flags": {r.key: {"us_per_launch": round(r.result["ms"] * 1e3, 3),
                                     "bitwise_vs_byte_form": r.result.get("bitwise_vs_byte_form")}
                             for r in rows if r.key.endswith("_packed")} or None},
        "configs": [row_json(r) for r in rows],
        "configs_split_depth": [row_json(r) for r in split_rows],
        "next_rows": [row_json(r) for r in next_rows],
        "workloads": [{k: ({kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                           if isinstance(v, dict) else (round(v, 2) if isinstance(v, float) else v))
                       for k, v in w.items()} for w in workloads],
        "workloads_note": WORKLOAD_NOTE,
        "full_rows": args.full_json,
    }
    full = json.dumps(out)
    try:
        os.makedirs(os.path.dirname(os.path.abspath(args.full_json)), exist_ok=True)
        with open(args.full_json, "w") as fh:
            fh.write(full + "\n")
    except OSError as e:
        log(f"full rows not written to {args.full_json}: {e}")
        out["full_rows"] = None
    log("full rows: " + full)
    print(compact_line(out, strict=False), flush=True)


if __name__ == "__main__":
    main()

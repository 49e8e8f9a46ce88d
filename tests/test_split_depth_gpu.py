"""The NNH_NUMERICS_SPLIT_DEPTH mode on the GPU: every product with m n <= 2^18 and k >= 256 is computed as
nn-cpp's depth cut computes its products (128-deep chains added in piece order). Each op is compared bit for bit
with the oracle switched to the same mode (whose split products are pinned to nn-cpp's own sgemm on each slab by
tests/test_oracle.py), and the GEMM with the north-star fp64 bound. Kernels that run whole-depth chains (the fused
attention forward, the LDS convolutions) must decline such products."""
import numpy as np
import pytest

from helpers import (UNDERFLOW_SHAPES, Problem, assert_same, bits_equal, first_diff, gpu_sgemm, oracle_sgemm,
                     underflow_problem, within_fp64_bound)
from nnh import synth

pytestmark = pytest.mark.gpu


@pytest.fixture
def split(gpu, oracle):
    import nnh
    prev = nnh.set_numerics(nnh.NUMERICS_SPLIT_DEPTH)
    oracle.set_numerics(1)
    try:
        yield
    finally:
        nnh.set_numerics(prev)
        oracle.set_numerics(0)


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_split_sgemm_matches_oracle(split, oracle, ta, tb):
    import nnh
    shapes = [(512, 512, 512), (64, 4096, 600), (256, 512, 784), (256, 10, 256), (33, 70, 300), (7, 9, 1100),
              (512, 513, 300), (100, 100, 255), (512, 512, 1200)]
    for i, (m, n, k) in enumerate(shapes):
        p = Problem(ta, tb, m, n, k, i % 2, 7000 + 10 * i + 2 * ta + tb)
        for acc in (0, 1):
            want = oracle_sgemm(oracle, p, acc)
            got = gpu_sgemm(p, acc)
            assert bits_equal(got, want), ((m, n, k), acc, first_diff(got, want))
            if i < 2:
                assert within_fp64_bound(got, p, acc, oracle)
    p = Problem(ta, tb, 40, 48, 600, 0, 7100)
    for cfg in range(len(nnh.gemm_configs())):
        got = gpu_sgemm(p, 0, config=cfg)
        assert bits_equal(got, oracle_sgemm(oracle, p, 0)), cfg


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_split_underflowing_chains_keep_negative_zero(split, oracle, ta, tb):
    """Pieces whose every product rounds to -0 are -0 and add to -0: the steps past a short last piece must
    leave -0 alone."""
    for m, n, k in UNDERFLOW_SHAPES + [(512, 512, 600), (64, 4096, 300)]:
        p = underflow_problem(ta, tb, m, n, k)
        for acc in (0, 1):
            want = oracle_sgemm(oracle, p, acc)
            assert np.all(np.signbit(want[:m, :n]))
            got = gpu_sgemm(p, acc)
            assert bits_equal(got, want), ((m, n, k), acc, first_diff(got, want))


def test_split_linear_mlp_matches_oracle(split, oracle):
    """BASELINE config 2's MLP forward and backward in split mode."""
    import torch

    import nnh
    dims = [784, 512, 256, 10]
    x = synth.mt19937_uniform(1, 256 * 784, 0.0, 1.0).reshape(256, 784)
    h = x
    for i in range(3):
        w = synth.mt19937_uniform(100 + i, dims[i + 1] * dims[i], -1 / np.sqrt(dims[i]), 1 / np.sqrt(dims[i])) \
            .reshape(dims[i + 1], dims[i])
        b = synth.mt19937_uniform(300 + i, dims[i + 1], -0.1, 0.1)
        y = host(nnh.linear_forward(dev(h), dev(w), dev(b), relu=True))
        want = oracle.relu(oracle.linear_forward(h, w, b))
        assert_same(y, want, ("forward", i))
        g = synth.normal(200 + i, (256, dims[i + 1]))
        dx, dw, db = torch.empty((256, dims[i]), device="cuda"), torch.empty(w.shape, device="cuda"), \
            torch.empty(dims[i + 1], device="cuda")
        nnh.linear_backward(dev(g), dev(h), dev(w), dx, True, dw, True, db, True)
        wdx, wdw, wdb = oracle.linear_backward(g, h, w)
        for got, wnt, name in ((dx, wdx, "dx"), (dw, wdw, "dw"), (db, wdb, "db")):
            assert_same(host(got), wnt, (name, i))
        h = y


def test_split_attention_and_conv_match_oracle(split, oracle):
    """Attention with 256 keys (its O = P V product now splits, so the fused kernel declines) and a convolution
    whose products split (288 deep), forward and backward."""
    import torch

    import nnh
    q, k, v, g = (synth.normal(60 + i, (2, 256, 128)) for i in range(4))
    out, probs = nnh.attention_forward(dev(q), dev(k), dev(v), 2)
    wout, wprobs = oracle.attention_forward(q, k, v, 2)
    assert_same(host(out), wout, "attention out")
    assert_same(host(probs), wprobs, "attention probs")
    dq, dk, dv = (torch.empty((2, 256, 128), device="cuda") for _ in range(3))
    nnh.attention_backward(dev(g), dev(q), dev(k), dev(v), probs, 2, None, False, dq, True, dk, True, dv, True)
    for got, want, name in zip((dq, dk, dv), oracle.attention_backward(g, q, k, v, wprobs, 2), ("dq", "dk", "dv")):
        assert_same(host(got), want, name)
    x = synth.mt19937_uniform(70, 4 * 32 * 14 * 14, 0.0, 1.0).reshape(4, 32, 14, 14)
    w = synth.normal(71, (64, 32, 3, 3)) * np.float32(0.05)
    b = synth.mt19937_uniform(72, 64, -0.1, 0.1)
    y, alive = nnh.conv2d_forward(dev(x), dev(w.astype(np.float32)), dev(b), 1, 1, True)
    wy, wal = oracle.conv2d_forward(x, w.astype(np.float32), b, 1, 1, True)
    assert_same(host(y), wy, "conv y")
    gr = synth.normal(73, wy.shape)
    dx, dw, db = torch.empty(x.shape, device="cuda"), torch.empty(w.shape, device="cuda"), torch.empty(64, device="cuda")
    nnh.conv2d_backward(dev(gr), dev(x), dev(w.astype(np.float32)), alive, 1, 1, dx, True, dw, True, db, True)
    wdx, wdw, wdb = oracle.conv2d_backward(gr, x, w.astype(np.float32), wal, 1, 1)
    for got, want, name in ((dx, wdx, "dx"), (dw, wdw, "dw"), (db, wdb, "db")):
        assert_same(host(got), want, name)


def test_split_mode_is_reset_and_rejected_values(gpu):
    import nnh
    assert nnh.lib().nnh_get_numerics() == nnh.NUMERICS_NNCPP
    assert nnh.lib().nnh_set_numerics(7) == nnh.ERR_INVALID


def test_two_streams_in_two_modes_at_once(gpu, oracle):
    """A stream's own mode: two streams, one per mode, issue the same products from two threads at once; each
    stream's outputs are its mode's bits (the oracle in that mode), and the process default is left as it was."""
    import threading

    import torch

    import nnh
    shapes = [(512, 512, 512), (64, 4096, 600), (256, 256, 512)]
    probs = [Problem(0, 1, m, n, k, 0, 7300 + i) for i, (m, n, k) in enumerate(shapes)]
    want = {}
    for mode in (0, 1):
        oracle.set_numerics(mode)
        want[mode] = [oracle_sgemm(oracle, p, 0) for p in probs]
    oracle.set_numerics(0)
    assert not all(bits_equal(want[0][i], want[1][i]) for i in range(len(probs)))
    streams = {0: torch.cuda.Stream(), 1: torch.cuda.Stream()}
    nnh.set_stream_numerics(nnh.NUMERICS_NNCPP, streams[0])
    nnh.set_stream_numerics(nnh.NUMERICS_SPLIT_DEPTH, streams[1])
    default = nnh.lib().nnh_get_numerics()
    try:
        assert nnh.get_stream_numerics(streams[1]) == nnh.NUMERICS_SPLIT_DEPTH
        ops = {mode: [(torch.from_numpy(p.a).cuda(), torch.from_numpy(p.b).cuda(), torch.empty((p.m, p.ldc),
                                                                                                   device="cuda"))
                      for p in probs] for mode in (0, 1)}
        torch.cuda.synchronize()
        errors = []

        def issue(mode):
            try:
                with torch.cuda.stream(streams[mode]):
                    for rep in range(20):
                        for p, (a, b, c) in zip(probs, ops[mode]):
                            nnh.sgemm(p.ta, p.tb, p.m, p.n, p.k, a, p.lda, b, p.ldb, c, p.ldc, 0,
                                      stream=streams[mode])
            except Exception as e:  # reported by the main thread
                errors.append(e)

        threads = [threading.Thread(target=issue, args=(mode,)) for mode in (0, 1)]
        for t in threads:
            t.start()
        for t in threads:
            t.join()
        torch.cuda.synchronize()
        assert not errors, errors
        for mode in (0, 1):
            for i, (p, (_, _, c)) in enumerate(zip(probs, ops[mode])):
                assert bits_equal(host(c), want[mode][i][: p.m]), (mode, shapes[i])
        assert nnh.lib().nnh_get_numerics() == default
    finally:
        nnh.set_stream_numerics(nnh.NUMERICS_DEFAULT, streams[0])
        nnh.set_stream_numerics(nnh.NUMERICS_DEFAULT, streams[1])
    assert nnh.get_stream_numerics(streams[1]) == default

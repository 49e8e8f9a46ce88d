"""nn::hip (include/nn_hip.hpp): nn-cpp's op surface on device-resident tensors, run through a C harness
(tests/cpp/nn_hip_harness.cpp) and compared bit for bit with the same graphs built from nn-cpp's own ops on its CPU
build (oracle/ref_shim.cpp): nn-cpp's cnn_mnist model (conv2d_relu, maxpool2d, reshape, linear, relu), an MLP, a
batched matmul into a folded matmul_bt, self-attention (one node as q, k and v), the masked softmax, forward and
backward; and the TensorShapeError cases. Between the copy in and the copy out every op reads and writes HBM."""
import ctypes as C
import os

import numpy as np
import pytest

from helpers import assert_same
from nnh import synth

pytestmark = pytest.mark.gpu

HARNESS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "lib", "libnn_hip_harness.so")
_f = C.POINTER(C.c_float)
_sz = C.c_size_t


def fp(a):
    return None if a is None else a.ctypes.data_as(_f)


def ptrs(arrs):
    return (_f * len(arrs))(*[fp(a) for a in arrs])


@pytest.fixture(scope="module")
def harness(gpu):
    if not os.path.exists(HARNESS):
        pytest.fail(f"{HARNESS} missing: build it with `make -C tests/cpp` (or __graft_entry__.build())")
    return C.CDLL(HARNESS)


def uni(seed, shape, bound):
    return np.ascontiguousarray(synth.mt19937_uniform(seed, int(np.prod(shape)), -bound, bound).reshape(shape))


@pytest.mark.parametrize("fused", [0, 1])
@pytest.mark.parametrize("dims", [(32, 1, 28, 8, 16, 128, 10), (3, 2, 12, 5, 7, 9, 4)])
def test_cnn_step_matches_nncpp(harness, ref, dims, fused):
    """nn-cpp's cnn_mnist (apps/bench/workloads.cpp:113-137): N 32, 1 x 28 x 28, conv 8 and 16, hidden 128; fused:
    each conv2d_relu -> maxpool2d pair as nn::hip::conv2d_relu_maxpool2d (the first layer in one pass)."""
    N, c0, side, c1, c2, hidden, classes = dims
    flat = c2 * (side // 4) ** 2
    shapes = [(c1, c0, 3, 3), (c1,), (c2, c1, 3, 3), (c2,), (hidden, flat), (hidden,), (classes, hidden), (classes,)]
    fans = [c0 * 9, c0 * 9, c1 * 9, c1 * 9, flat, flat, hidden, hidden]
    params = [uni(60 + i, s, 1 / np.sqrt(f)) for i, (s, f) in enumerate(zip(shapes, fans))]
    x = np.ascontiguousarray(synth.mt19937_uniform(59, N * c0 * side * side, 0, 1).reshape(N, c0, side, side))
    g = synth.normal(58, (N, classes))
    results = []
    for fn in (harness.h_cnn_step_fused if fused else harness.h_cnn_step, ref.lib.nnref_cnn_step):
        outs = [np.empty((N, classes), np.float32), np.empty_like(x)] + [np.empty_like(p) for p in params]
        rc = fn(fp(x), _sz(N), _sz(c0), _sz(side), _sz(c1), _sz(c2), _sz(hidden), _sz(classes), *[fp(p) for p in params],
                fp(g), *[fp(o) for o in outs])
        assert rc == 0, (fn, rc)
        results.append(outs)
    names = ["logits", "dx", "dw1", "db1", "dw2", "db2", "dw3", "db3", "dw4", "db4"]
    for name, got, want in zip(names, *results):
        assert_same(got, want, (name, dims, fused))


def test_mlp_step_matches_nncpp(harness, ref):
    """mlp_wide's model (784 -> 1024 -> 1024 -> 10 with ReLU between, workloads.cpp:100-107) at batch 256."""
    dims = [784, 1024, 1024, 10]
    M, L = 256, 3
    x = np.ascontiguousarray(synth.mt19937_uniform(70, M * 784, 0, 1).reshape(M, 784))
    ws = [uni(71 + i, (dims[i + 1], dims[i]), 1 / np.sqrt(dims[i])) for i in range(L)]
    bs = [uni(75 + i, (dims[i + 1],), 1 / np.sqrt(dims[i])) for i in range(L)]
    g = synth.normal(79, (M, 10))
    results = []
    for fn in (harness.h_mlp_step, ref.lib.nnref_mlp_step):
        y, dx = np.empty((M, 10), np.float32), np.empty_like(x)
        dws, dbs = [np.empty_like(w) for w in ws], [np.empty_like(b) for b in bs]
        rc = fn(fp(x), _sz(M), (C.c_size_t * 4)(*dims), L, ptrs(ws), ptrs(bs), fp(g), fp(y), fp(dx), ptrs(dws), ptrs(dbs))
        assert rc == 0, (fn, rc)
        results.append([y, dx] + dws + dbs)
    for i, (got, want) in enumerate(zip(*results)):
        assert_same(got, want, ("mlp", i))


def test_matmul_chain_matches_nncpp(harness, ref):
    """matmul_bt(matmul(a, b), c): a batched Value matmul into a folded matmul_bt, forward and backward."""
    a, b, c = uni(80, (3, 20, 30), 1), uni(81, (3, 30, 12), 1), uni(82, (7, 12), 1)
    g = synth.normal(83, (3, 20, 7))
    sh = lambda t: (C.c_size_t * t.ndim)(*t.shape)
    results = []
    for fn in (harness.h_matmul_chain, ref.lib.nnref_matmul_chain):
        outs = [np.empty((3, 20, 7), np.float32), np.empty_like(a), np.empty_like(b), np.empty_like(c)]
        assert fn(fp(a), sh(a), fp(b), sh(b), fp(c), sh(c), fp(g), *[fp(o) for o in outs]) == 0
        results.append(outs)
    for name, got, want in zip(["y", "da", "db", "dc"], *results):
        assert_same(got, want, name)


@pytest.mark.parametrize("causal", [0, 1])
def test_self_attention_matches_nncpp(harness, ref, causal):
    """attention(x, x, x): the one node's gradient is stored by dV, then dQ and dK add to it (ops.cpp:1274-1278)."""
    N, T, D, H = 2, 32, 64, 4
    x = synth.normal(90 + causal, (N, T, D))
    g = synth.normal(92, (N, T, D))
    results = []
    for fn in (harness.h_self_attention, ref.lib.nnref_self_attention):
        o, dx = np.empty_like(x), np.empty_like(x)
        assert fn(fp(x), _sz(N), _sz(T), _sz(D), _sz(H), causal, fp(g), fp(o), fp(dx)) == 0
        results.append([o, dx])
    for name, got, want in zip(["out", "dx"], *results):
        assert_same(got, want, (name, causal))


@pytest.mark.parametrize("case", [(2, 3, 5, 7, 0.5, True, 0), (1, 2, 6, 6, 0.125, False, 1), (2, 2, 6, 6, 1.0, True, 1)])
def test_softmax_matches_nncpp(harness, ref, case):
    N, H, Tq, Tk, scale, masked, causal = case
    x = synth.normal(95, (N, H, Tq, Tk))
    g = synth.normal(96, (N, H, Tq, Tk))
    pad = np.ones((N, Tk), np.float32) if masked else None
    if masked:
        pad[0, -2:] = 0
    results = []
    for fn in (harness.h_softmax, ref.lib.nnref_softmax_step):
        y, dx = np.empty_like(x), np.empty_like(x)
        assert fn(fp(x), _sz(N), _sz(H), _sz(Tq), _sz(Tk), C.c_float(scale), fp(pad), causal, fp(g), fp(y), fp(dx)) == 0
        results.append([y, dx])
    for name, got, want in zip(["y", "dx"], *results):
        assert_same(got, want, (name, case))


def test_shape_errors_throw_tensor_shape_error(harness):
    """matmul, linear, conv2d, maxpool2d, attention, batchnorm and layernorm with shapes nn-cpp rejects, and
    backward() on a non-scalar: each throws nn::hip::TensorShapeError."""
    assert harness.h_shape_errors() == 0x7FF


@pytest.mark.parametrize("dims", [(16, 1, 24, 8, 16, 7), (3, 2, 10, 5, 3, 4)])
def test_norm_step_matches_nncpp(harness, ref, dims):
    """conv2d -> batchnorm with the ReLU folded -> maxpool2d -> conv2d -> batchnorm -> relu -> reshape -> layernorm
    -> linear, forward and every gradient (the ops of nn-cpp's cnn_fer and transformer workloads), through nn::hip
    against nn-cpp's own ops."""
    N, c0, side, c1, c2, classes = dims
    flat = c2 * (side // 2) ** 2
    shapes = [(c1, c0, 3, 3), (c1,), (c1,), (c1,), (c2, c1, 3, 3), (c2,), (c2,), (c2,), (flat,), (flat,),
              (classes, flat), (classes,)]
    params = [uni(110 + i, s, 0.5) for i, s in enumerate(shapes)]
    for i in (2, 6, 8):  # scales near 1
        params[i] = (params[i] + 1).astype(np.float32)
    x = np.ascontiguousarray(synth.mt19937_uniform(109, N * c0 * side * side, 0, 1).reshape(N, c0, side, side))
    g = synth.normal(108, (N, classes))
    results = []
    for fn in (harness.h_norm_step, ref.lib.nnref_norm_step):
        y = np.empty((N, classes), np.float32)
        grads = [np.empty_like(p) for p in params]
        dx = np.empty_like(x)
        rc = fn(fp(x), _sz(N), _sz(c0), _sz(side), _sz(c1), _sz(c2), _sz(classes), ptrs(params), fp(g), fp(y),
                ptrs(grads), fp(dx))
        assert rc == 0, (fn, rc)
        results.append([y, dx] + grads)
    names = ["y", "dx", "dw1", "db1", "dbn1_w", "dbn1_b", "dw2", "db2", "dbn2_w", "dbn2_b", "dln_g", "dln_b", "dw3",
             "db3"]
    for name, got, want in zip(names, *results):
        assert_same(got, want, (name, dims))

"""The module layer over device tensors (include/nn_hip_modules.hpp): nn-cpp's Sequential, Conv2d, Linear,
MaxPool2d, Flatten, ReLU, Dropout, MultiHeadAttention and Transformer built with nn::hip after nn::hip::manual_seed,
against the same models built by nn-cpp's CPU build after nn::manual_seed (oracle/ref_shim.cpp's nnref_module_run):
the initial parameters (from the seeded Tensor::random stream), the output and every gradient must be bit-identical.
The reference's own tests of these modules: tests/test_nn.cpp:587-651, tests/test_transformer.cpp:149-276.

The seeding itself (include/nn/random.hpp, src/random.cpp) is host code and is checked without a GPU."""
import ctypes as C
import os

import numpy as np
import pytest

from helpers import assert_same
from nnh import synth

HARNESS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "lib", "libnn_hip_harness.so")


@pytest.fixture(scope="module")
def harness():
    # torch's HIP runtime first, as every GPU test has it (the harness library brings the ROCm runtime it was built
    # against; a process that loads it before torch initialises finds no device)
    import torch
    torch.cuda.is_available()
    if not os.path.exists(HARNESS):
        pytest.fail(f"{HARNESS} missing: build it with `make -C tests/cpp` (or __graft_entry__.build())")
    return C.CDLL(HARNESS)


@pytest.mark.parametrize("seed,stream,gens", [(1234, "tensor.random", 1), (7, "dropout", 3), (2 ** 63 + 5, "x", 2)])
def test_derived_generators_match_nncpp(harness, ref, seed, stream, gens):
    """derive_generator's k-th generator of a named stream after manual_seed: splitmix64 of the seed, FNV-1a of the
    name and k, through std::seed_seq into std::mt19937 (src/random.cpp), the same 32-bit draws as nn-cpp's."""
    n = 600
    want, got = np.zeros(n, np.uint32), np.zeros(n, np.uint32)
    u32p = C.POINTER(C.c_uint32)
    for lib, fn, out in ((ref.lib, "nnref_random_draws", want), (harness, "h_random_draws", got)):
        f = getattr(lib, fn)
        f.argtypes = [C.c_ulonglong, C.c_char_p, C.c_int, C.c_size_t, u32p]
        assert f(seed, stream.encode(), gens, n, out.ctypes.data_as(u32p)) == 0
    assert np.array_equal(got, want)
    assert len(set(got.tolist())) > n // 2  # not a constant stream


# (model, input shape, output shape, ids vocabulary or None): see nnref_module_run in oracle/ref_shim.cpp
MODELS = [
    (0, (32, 1, 28, 28), (32, 10), None),   # cnn_mnist: Conv2d + ReLU (+ MaxPool2d) folded, Flatten, Linear
    (1, (2, 16, 64), (2, 16, 64), None),    # MultiHeadAttention, causal: the fused attention op
    (3, (4, 6, 20), (4, 6, 5), None),       # Linear on a 3-D input, ReLU, Linear
    (4, (2, 7), (2, 7, 11), 11),            # Transformer: learned positions (slice), two causal blocks
    (5, (4, 6, 20), (4, 6, 5), None),       # Dropout(0.25) in training mode between the Linears (mask, mul)
    (6, (3, 9), (3, 9, 13), 13),            # Transformer in evaluation mode: dropout off, sinusoidal, non-causal
]


@pytest.mark.gpu
@pytest.mark.parametrize("which,xshape,yshape,vocab", MODELS)
def test_modules_match_nncpp(gpu, harness, ref, which, xshape, yshape, vocab):
    n = int(np.prod(xshape))
    if vocab:
        x = (np.arange(n, dtype=np.int64) * 7 % vocab).astype(np.float32).reshape(xshape)
    else:
        x = synth.mt19937_uniform(50 + which, n, 0.0, 1.0).reshape(xshape)
    g = synth.normal(60 + which, yshape)
    o_ref, g_ref = ref.module_run(which, 4321, x, g)
    cap_o, cap_g = 1 << 20, 1 << 22
    out, grads = np.empty(cap_o, np.float32), np.empty(cap_g, np.float32)
    n_out, n_grads = C.c_size_t(0), C.c_size_t(0)
    fp = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))
    xc, gc = np.ascontiguousarray(x, np.float32), np.ascontiguousarray(g, np.float32)
    rc = harness.h_module_run(which, 4321, fp(xc), (C.c_size_t * x.ndim)(*x.shape), x.ndim, fp(gc), fp(out),
                              C.c_size_t(cap_o), fp(grads), C.c_size_t(cap_g), C.byref(n_out), C.byref(n_grads))
    harness.h_last_error.restype = C.c_char_p
    assert rc == 0, (rc, harness.h_last_error().decode())
    assert n_out.value == o_ref.size and n_grads.value == g_ref.size
    assert_same(out[: n_out.value], o_ref, ("output", which))
    assert_same(grads[: n_grads.value], g_ref, ("gradients", which))


@pytest.mark.gpu
@pytest.mark.parametrize("count,same", [(1, 0), (1000, 0), (70001, 1)])
def test_mul_op_bitwise(gpu, harness, count, same):
    """nn::hip::mul (ops.cpp:347-357, the op Dropout multiplies its mask in with): y = a * b; each operand's
    gradient is g * (the other) + 0 when fresh, and one node as both operands takes g * a + 0, then adds g * a. A
    float32 product is correctly rounded, so numpy gives the reference's bits; signed zeros, Inf and NaN included."""
    rng = np.random.default_rng(count)
    a = rng.standard_normal(count).astype(np.float32)
    b = rng.standard_normal(count).astype(np.float32)
    g = rng.standard_normal(count).astype(np.float32)
    if count > 8:
        a[:4] = [0.0, -0.0, np.inf, np.nan]
        b[4:8] = [-0.0, 0.0, -np.inf, 1e-38]
        g[8:10] = [-0.0, 0.0]
    y, da, db = (np.empty(count, np.float32) for _ in range(3))
    fp = lambda x: x.ctypes.data_as(C.POINTER(C.c_float))
    rc = harness.h_mul_step(fp(a), fp(b), C.c_size_t(count), same, fp(g), fp(y), fp(da), fp(db))
    assert rc == 0, rc
    zero = np.float32(0.0)
    with np.errstate(all="ignore"):
        if same:
            t = g * a
            assert_same(y, a * a, "y", nan_equal=True)
            assert_same(da, (t + zero) + t, "da", nan_equal=True)
        else:
            assert_same(y, a * b, "y", nan_equal=True)
            assert_same(da, g * b + zero, "da", nan_equal=True)
            assert_same(db, g * a + zero, "db", nan_equal=True)

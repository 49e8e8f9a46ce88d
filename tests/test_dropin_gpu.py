"""The drop-in, literally: nn-cpp's own unmodified sources, compiled with their src/kernels/gemm.cpp left out and
this project's nn::kernels::sgemm (lib/libnn_gemm_hip.so, host pointers, GPU underneath) linked in its place
(oracle/_ref/libnnref_hip.so). The reference's matmul, linear, conv2d_relu and attention, forward and backward,
then run with every GEMM on the MI355X, and must give the bits of nn-cpp's CPU build.
"""
import ctypes as C
import os

import numpy as np
import pytest

from helpers import assert_same
from nnh import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def refs(gpu):
    from pyoracle import REF_HIP_SO, REF_SO, Reference
    if not (os.path.exists(REF_SO) and os.path.exists(REF_HIP_SO)):
        pytest.skip("nn-cpp builds under oracle/_ref missing (built by __graft_entry__.build() where /root/reference exists)")
    import nnh
    cpu, hip = Reference(REF_SO), Reference(REF_HIP_SO)
    calls = nnh.host_lib().nnh_sgemm_host_calls
    calls.restype = C.c_ulonglong
    return cpu, hip, calls


def same(got, want, what):
    assert_same(got, want, what)


def test_sgemm_symbol_is_the_gpu_one(refs):
    cpu, hip, calls = refs
    a, b = synth.uniform_operands(1, [(300, 200), (200, 100)])
    c = np.zeros((300, 100), np.float32)
    before = calls()
    got = hip.sgemm(0, 0, 300, 100, 200, a, 200, b, 100, c, 100, 0)
    assert calls() == before + 1, "the nn-cpp build did not route its GEMM to the GPU drop-in"
    same(got, cpu.sgemm(0, 0, 300, 100, 200, a, 200, b, 100, c, 100, 0), "sgemm")


def test_nncpp_ops_on_the_gpu_give_nncpp_bits(refs):
    cpu, hip, calls = refs
    before = calls()
    # Tensor matmul with broadcasting and transposes
    a, b = synth.uniform_operands(2, [(2, 3, 33, 65), (1, 3, 129, 65)])
    for r in (cpu, hip):
        r.set_threads(4)
    rc1, m1 = cpu.matmul(a, b, False, True)
    rc2, m2 = hip.matmul(a, b, False, True)
    assert rc1 == rc2 == 0
    same(m2, m1, "matmul")
    # linear forward/backward (BASELINE config 2's first layer)
    x = synth.mt19937_uniform(1, 256 * 784, 0.0, 1.0).reshape(256, 784)
    w = synth.mt19937_uniform(100, 512 * 784, -1 / 28, 1 / 28).reshape(512, 784)
    bias = np.zeros(512, np.float32)
    g = synth.normal(200, (256, 512))
    same(hip.linear_forward(x, w, bias), cpu.linear_forward(x, w, bias), "linear forward")
    for p, q, key in zip(hip.linear_backward(x, w, bias, g), cpu.linear_backward(x, w, bias, g), ("dx", "dw", "db")):
        same(p, q, "linear " + key)
    # conv2d_relu forward/backward
    xc = synth.mt19937_uniform(2, 8 * 3 * 20 * 20, 0.0, 1.0).reshape(8, 3, 20, 20)
    wc = synth.normal(21, (16, 3, 3, 3))
    bc = synth.mt19937_uniform(3, 16)
    gc = synth.normal(22, (8, 16, 20, 20))
    same(hip.conv2d_forward(xc, wc, bc, 1, 1, 1), cpu.conv2d_forward(xc, wc, bc, 1, 1, 1), "conv2d_relu forward")
    for p, q, key in zip(hip.conv2d_backward(xc, wc, bc, 1, 1, 1, gc), cpu.conv2d_backward(xc, wc, bc, 1, 1, 1, gc),
                         ("dx", "dw", "db")):
        same(p, q, "conv2d_relu " + key)
    # attention forward/backward, causal with padding: the softmax runs in nn-cpp's code on both sides
    q, k, v, ga = (synth.normal(40 + i, (4, 32, 64)) for i in range(4))
    mask = np.ones((4, 32), np.float32)
    mask[2, 25:] = 0
    same(hip.attention_forward(q, k, v, 4, mask, True), cpu.attention_forward(q, k, v, 4, mask, True), "attention")
    for p_, q_, key in zip(hip.attention_backward(q, k, v, 4, ga, mask, True),
                           cpu.attention_backward(q, k, v, 4, ga, mask, True), ("dq", "dk", "dv")):
        same(p_, q_, "attention " + key)
    assert calls() > before + 10


def test_host_entry_point_matches_oracle(gpu, oracle):
    """nnh_sgemm_host (the C entry of the drop-in) on padded host buffers, all flags."""
    import nnh
    from helpers import Problem
    seed = 600
    for ta in (0, 1):
        for tb in (0, 1):
            for acc in (0, 1):
                p = Problem(ta, tb, 70, 90, 300, 3, seed)
                seed += 1
                c = p.c.copy()
                nnh.sgemm_host(ta, tb, p.m, p.n, p.k, p.a, p.lda, p.b, p.ldb, c, p.ldc, acc)
                same(c, oracle.sgemm(ta, tb, p.m, p.n, p.k, p.a, p.lda, p.b, p.ldb, p.c, p.ldc, acc), (ta, tb, acc))


# (model, input shape, output shape): nn-cpp's modules, unchanged, through the drop-in (see nnref_module_run)
MODULES = [
    (0, (32, 1, 28, 28), (32, 10)),   # cnn_mnist: Sequential folds Conv2d + ReLU into conv2d_relu
    (1, (2, 16, 64), (2, 16, 64)),    # MultiHeadAttention, causal, no dropout: the fused attention op
    (2, (2, 16, 64), (2, 16, 64)),    # MultiHeadAttention with dropout in training: the composed path
    (3, (4, 6, 20), (4, 6, 5)),       # Linear on a 3-D input, ReLU, Linear
]


@pytest.mark.parametrize("which,xshape,yshape", MODULES)
def test_modules_run_unchanged_through_the_dropin(refs, which, xshape, yshape):
    """src/nn/{sequential,conv2d,linear,pool2d,activation,attention,dropout}.cpp compiled with the drop-in in place of
    gemm.cpp: the output and every parameter's and the input's gradient bit-identical to nn-cpp's CPU build, with
    the modules' GEMMs run on the GPU (the reference's own tests of these callers: tests/test_nn.cpp:587-651,
    tests/test_transformer.cpp:149-276)."""
    cpu, hip, calls = refs
    x = synth.mt19937_uniform(30 + which, int(np.prod(xshape)), 0.0, 1.0).reshape(xshape)
    g = synth.normal(40 + which, yshape)
    before = calls()
    o_cpu, g_cpu = cpu.module_run(which, 1234, x, g)
    o_hip, g_hip = hip.module_run(which, 1234, x, g)
    assert calls() > before, "the module's products did not reach the GPU"
    same(o_hip, o_cpu, ("output", which))
    same(g_hip, g_cpu, ("gradients", which))


def test_portable_and_unpacked_kernels_through_the_dropin(refs):
    """tests/test_kernels.cpp:157-167's sweep (sizes {1, 7, 33, 257}^3, both transposes, accumulate) for the
    drop-in's sgemm_portable and sgemm_unpacked: the GPU computes nn-cpp's AVX2 chain for every entry point, so
    each is bit-identical to nn-cpp's sgemm, and within the reference test's tolerance (1e-5 of sum |a b|, floor
    1e-6; test_kernels.cpp:101-146) of nn-cpp's own portable and unpacked kernels."""
    from helpers import Problem
    cpu, hip, calls = refs
    sizes = (1, 7, 33, 257)
    seed = 1
    for ta in (0, 1):
        for tb in (0, 1):
            for acc in (0, 1):
                for m in sizes:
                    for n in sizes:
                        for k in sizes:
                            p = Problem(ta, tb, m, n, k, 0, seed)
                            seed += 1
                            args = (ta, tb, m, n, k, p.a, p.lda, p.b, p.ldb, p.c, p.ldc, acc)
                            want = cpu.sgemm(*args)
                            opa, opb = (p.a.T if ta else p.a)[:m, :k], (p.b.T if tb else p.b)[:k, :n]
                            mag = np.abs(opa.astype(np.float64)) @ np.abs(opb.astype(np.float64))
                            if acc:
                                mag = mag + np.abs(p.c[:m, :n])
                            tol = np.maximum(1e-5 * mag, 1e-6)
                            for name in ("portable", "unpacked"):
                                got = hip.sgemm_variant(name, *args)
                                same(got, want, (name, ta, tb, acc, m, n, k))
                                theirs = cpu.sgemm_variant(name, *args)
                                assert np.all(np.abs(got[:m, :n].astype(np.float64) - theirs[:m, :n]) <= tol), \
                                    (name, ta, tb, acc, m, n, k)

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

"""nn-cpp's bench models end to end: one training step (forward, zero_grad, backward from a fixed gradient of the
logits) through nn::hip on the GPU (lib/libnnh_workloads.so) against nn-cpp's own step on the CPU
(oracle/_ref/libnnref.so, its compiled sources), on make_workload's seeded data: the logits and every parameter's
gradient bit for bit. transformer_tiny runs nn-cpp's own Transformer module on the CPU side, so the GPU graph's
composition (embedding, sinusoidal positions, pre-norm blocks with fused attention and GELU MLP, final LayerNorm and
head) is checked against the reference's modules, not restated. Two steps in a row check that zero_grad and the
fresh-gradient rules leave nothing behind."""
import ctypes as C
import os

import numpy as np
import pytest

from helpers import assert_same

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def wlib(gpu):
    return C.CDLL(os.path.join(ROOT, "nn-cpp_amd", "lib", "libnnh_workloads.so"))


@pytest.mark.parametrize("name", ["mlp_wide", "cnn_mnist", "transformer_tiny"])
def test_workload_step_matches_nncpp(wlib, ref, name):
    from nnh import workloads as wl
    w = wl.by_name(name)
    params, x, g = wl.inputs(w, 1)
    rc, _, _, want_logits, want_grads = wl.run_step(ref.lib.nnref_time_workload_step, w, params, x, g, 0, 1, True)
    assert rc == 0
    rc, fwd, bwd, logits, grads = wl.run_step(wlib.nnh_bench_workload_step, w, params, x, g, 1, 1, True)
    assert rc == 0
    assert fwd[0] > 0 and bwd[0] > 0
    assert_same(logits, want_logits, f"{name} logits")
    for i, (a, b) in enumerate(zip(grads, want_grads)):
        assert_same(a, b, f"{name} grad of parameter {i} {w.shapes[i]}")


def test_transformer_tiny_nontrivial_norms_and_biases(wlib, ref):
    """Another seed, with every gamma, beta and bias drawn at random (make_workload leaves them at one and zero,
    which would hide a misplaced scale or shift)."""
    from nnh import workloads as wl
    w = wl.by_name("transformer_tiny")
    params, x, g = wl.inputs(w, 7)
    rng = np.random.default_rng(7)
    params = [p if p.ndim >= 2 else rng.uniform(0.5, 1.5, p.shape).astype(np.float32) if i in w.ones
              else rng.uniform(-0.5, 0.5, p.shape).astype(np.float32) for i, p in enumerate(params)]
    rc, _, _, want_logits, want_grads = wl.run_step(ref.lib.nnref_time_workload_step, w, params, x, g, 0, 1, True)
    assert rc == 0
    rc, _, _, logits, grads = wl.run_step(wlib.nnh_bench_workload_step, w, params, x, g, 0, 1, True)
    assert rc == 0
    assert_same(logits, want_logits, "logits")
    for i, (a, b) in enumerate(zip(grads, want_grads)):
        assert_same(a, b, f"grad of parameter {i}")

"""Writes tests/golden/reference_vectors.npz: outputs of nn-cpp itself (its unmodified sources compiled by
oracle/Makefile into oracle/_ref/libnnref.so) on small seeded cases.

Inputs are not stored: every case regenerates them from its seed with nnh.synth.mt19937_uniform, which
tests/test_oracle.py pins bit for bit to std::mt19937 + std::uniform_real_distribution<float>. Only the
reference's outputs are stored, so the fixture is data (expected values), a few hundred KB at most.

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "nn-cpp_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, HERE)

from golden_cases import (ATTENTION_CASES, BATCHNORM_CASES, CONV_CASES, LAYERNORM_CASES, LINEAR_CASES,  # noqa: E402
                          MATMUL_CASES, POOL_CASES, SGEMM_CASES, attention_inputs, batchnorm_inputs, conv_inputs,
                          layernorm_inputs, linear_inputs, matmul_inputs, pool_inputs, sgemm_inputs)
from pyoracle import Reference  # noqa: E402


def main():
    ref = Reference()
    ref.set_threads(8)
    out = {}
    for case in SGEMM_CASES:
        name, (ta, tb, m, n, k, acc, pad, seed) = case
        a, lda, b, ldb, c, ldc = sgemm_inputs(*case[1])
        out[f"sgemm/{name}"] = ref.sgemm(ta, tb, m, n, k, a, lda, b, ldb, c, ldc, acc)
    for name, spec in MATMUL_CASES:
        a, b, ta, tb = matmul_inputs(spec)
        rc, r = ref.matmul(a, b, ta, tb)
        assert rc == 0, name
        out[f"matmul/{name}"] = r
    for name, spec in LINEAR_CASES:
        x, w, bias, g = linear_inputs(spec)
        out[f"linear/{name}/y"] = ref.linear_forward(x, w, bias)
        dx, dw, db = ref.linear_backward(x, w, bias, g)
        out[f"linear/{name}/dx"], out[f"linear/{name}/dw"], out[f"linear/{name}/db"] = dx, dw, db
    for name, spec in CONV_CASES:
        x, w, bias, g, stride, pad, relu = conv_inputs(spec)
        out[f"conv/{name}/y"] = ref.conv2d_forward(x, w, bias, stride, pad, relu)
        dx, dw, db = ref.conv2d_backward(x, w, bias, stride, pad, relu, g)
        out[f"conv/{name}/dx"], out[f"conv/{name}/dw"], out[f"conv/{name}/db"] = dx, dw, db
    for name, spec in ATTENTION_CASES:
        q, k, v, heads, mask, causal, g = attention_inputs(spec)
        out[f"attention/{name}/out"] = ref.attention_forward(q, k, v, heads, mask, causal)
        dq, dk, dv = ref.attention_backward(q, k, v, heads, g, mask, causal)
        out[f"attention/{name}/dq"], out[f"attention/{name}/dk"], out[f"attention/{name}/dv"] = dq, dk, dv
    for name, spec in POOL_CASES:
        x, g, k, s = pool_inputs(spec)
        rc, y, dx = ref.maxpool2d(x, k, s, g)
        assert rc == 0, name
        out[f"pool/{name}/y"], out[f"pool/{name}/dx"] = y, dx
    for name, spec in BATCHNORM_CASES:
        x, w, b, g, relu = batchnorm_inputs(spec)
        rc, y, mean, var, (dx, dw, db) = ref.batchnorm(x, w, b, 1e-5, relu, g=g)
        assert rc == 0, name
        for key, val in (("y", y), ("mean", mean), ("var", var), ("dx", dx), ("dw", dw), ("db", db)):
            out[f"batchnorm/{name}/{key}"] = val
    for name, spec in LAYERNORM_CASES:
        x, gm, bt, g = layernorm_inputs(spec)
        D = x.shape[-1]
        rc, y, (dx, dg, db) = ref.layernorm(x.reshape(-1, D), gm, bt, 1e-5, g=g.reshape(-1, D))
        assert rc == 0, name
        for key, val in (("y", y.reshape(x.shape)), ("dx", dx.reshape(x.shape)), ("dgamma", dg), ("dbeta", db)):
            out[f"layernorm/{name}/{key}"] = val
    path = os.path.join(HERE, "reference_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {len(out)} arrays to {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()

"""Pins the oracle (CPU, no GPU): the C restatement of nn-cpp must be right before it can judge the GPU.

Each restated function is checked against at least one of: nn-cpp's own outputs (golden vectors written from
its compiled sources, and the compiled library itself when present), hand values from the reference's
tests, exact integer arithmetic, an fp64 closed form with the north-star bound, or an algebraic identity
(transposes, adjointness). The checks are chosen so a dropped term, a swapped index or a wrong flag fails.
"""
import os
import re
import subprocess
import sys

import numpy as np
import pytest

from helpers import UNDERFLOW_SHAPES, underflow_problem

from nnh import synth

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "reference_vectors.npz")


def golden():
    import sys
    sys.path.insert(0, os.path.join(HERE, "golden"))
    import golden_cases
    return golden_cases, np.load(GOLDEN, allow_pickle=False)


# ---------------------------------------------------------------- inputs

def test_mt19937_raw_stream_is_the_standard_one():
    """[rand.predef]: the 10000th output of a default-constructed std::mt19937 (seed 5489) is 4123659995."""
    assert int(synth.mt19937_raw(5489, 10000)[-1]) == 4123659995


@pytest.mark.parametrize("seed,lo,hi", [(0, -1.0, 1.0), (1, 0.0, 1.0), (4, -1.0, 1.0), (2, -0.3, 0.3), (99, -2.0, 2.0)])
def test_uniform_stream_matches_libstdcxx(oracle, seed, lo, hi):
    """nnh.synth reproduces std::uniform_real_distribution<float> over std::mt19937 bit for bit."""
    assert synth.mt19937_uniform(seed, 200000, lo, hi).tobytes() == oracle.mt19937_uniform(seed, lo, hi, 200000).tobytes()


# ---------------------------------------------------------------- golden vectors (nn-cpp's own outputs)

def test_golden_sgemm(oracle):
    gc, g = golden()
    for name, spec in gc.SGEMM_CASES:
        ta, tb, m, n, k, acc, pad, seed = spec
        a, lda, b, ldb, c, ldc = gc.sgemm_inputs(*spec)
        got = oracle.sgemm(ta, tb, m, n, k, a, lda, b, ldb, c, ldc, acc)
        assert got.tobytes() == g[f"sgemm/{name}"].tobytes(), name


def test_golden_linear(oracle):
    gc, g = golden()
    for name, spec in gc.LINEAR_CASES:
        x, w, bias, gr = gc.linear_inputs(spec)
        assert oracle.linear_forward(x, w, bias).tobytes() == g[f"linear/{name}/y"].tobytes(), name
        # leaves accumulate into zeroed gradients (first == false), as in a training step
        dx, dw, db = oracle.linear_backward(gr, x, w, dx_first=False, dw_first=False, db_first=False)
        for key, arr in (("dx", dx), ("dw", dw), ("db", db)):
            assert arr.tobytes() == g[f"linear/{name}/{key}"].tobytes(), (name, key)


def test_golden_conv(oracle):
    gc, g = golden()
    for name, spec in gc.CONV_CASES:
        x, w, bias, gr, stride, pad, relu = gc.conv_inputs(spec)
        y, alive = oracle.conv2d_forward(x, w, bias, stride, pad, relu)
        assert y.tobytes() == g[f"conv/{name}/y"].tobytes(), name
        dx, dw, db = oracle.conv2d_backward(gr, x, w, alive if relu else None, stride, pad)
        for key, arr in (("dx", dx), ("dw", dw), ("db", db)):
            assert arr.tobytes() == g[f"conv/{name}/{key}"].tobytes(), (name, key)


def test_golden_attention(oracle):
    gc, g = golden()
    for name, spec in gc.ATTENTION_CASES:
        q, k, v, heads, mask, causal, gr = gc.attention_inputs(spec)
        out, probs = oracle.attention_forward(q, k, v, heads, mask, causal)
        assert out.tobytes() == g[f"attention/{name}/out"].tobytes(), name
        dq, dk, dv = oracle.attention_backward(gr, q, k, v, probs, heads, mask, causal)
        for key, arr in (("dq", dq), ("dk", dk), ("dv", dv)):
            assert arr.tobytes() == g[f"attention/{name}/{key}"].tobytes(), (name, key)


def test_golden_matmul_against_batched_sgemm(oracle):
    """nn::matmul's batching (broadcast, fold) as per-matrix oracle sgemm calls reproduces nn-cpp's bits."""
    gc, g = golden()
    for name, spec in gc.MATMUL_CASES:
        a, b, ta, tb = gc.matmul_inputs(spec)
        want = g[f"matmul/{name}"]
        assert oracle_matmul(oracle, a, b, ta, tb).tobytes() == want.tobytes(), name


def oracle_matmul(oracle, a, b, ta, tb):
    """nn::matmul (src/tensor.cpp:571-641) composed from oracle sgemm calls."""
    a_rows, a_cols = a.shape[-2:]
    b_rows, b_cols = b.shape[-2:]
    m, k = (a_cols, a_rows) if ta else (a_rows, a_cols)
    n = b_rows if tb else b_cols
    if b.ndim == 2 and not ta and a.ndim > 2:
        M = a.size // a_cols
        out = np.zeros(a.shape[:-1] + (n,), np.float32)
        return oracle.sgemm(0, tb, M, n, k, a, a_cols, b, b_cols, out.reshape(M, n), n, 0).reshape(out.shape)
    batch = np.broadcast_shapes(a.shape[:-2], b.shape[:-2])
    out = np.zeros(batch + (m, n), np.float32)
    ab = np.broadcast_to(a, batch + a.shape[-2:])
    bb = np.broadcast_to(b, batch + b.shape[-2:])
    for idx in np.ndindex(*batch):
        out[idx] = oracle.sgemm(ta, tb, m, n, k, np.ascontiguousarray(ab[idx]), a_cols, np.ascontiguousarray(bb[idx]),
                                b_cols, out[idx], n, 0)
    return out


# ---------------------------------------------------------------- the compiled reference itself

def test_oracle_sgemm_matches_nncpp_sweep(oracle, ref):
    """Random sweep of shapes, flags, accumulate and ld padding, including depth-cut shapes: bit-identical."""
    rng = np.random.default_rng(7)
    sizes = (1, 2, 7, 33, 64, 129, 257)
    cases = [(int(rng.choice(sizes)), int(rng.choice(sizes)), int(rng.choice(sizes))) for _ in range(24)]
    cases += [(64, 64, 1024), (40, 48, 589), (7, 300, 768), (64, 64, 511), (300, 300, 512), (5, 9, 1100)]
    seed = 100
    for (m, n, k) in cases:
        for ta in (0, 1):
            for tb in (0, 1):
                for acc in (0, 1):
                    spec = (ta, tb, m, n, k, acc, int(rng.integers(0, 4)), seed)
                    seed += 1
                    import golden_cases as gc
                    a, lda, b, ldb, c, ldc = gc.sgemm_inputs(*spec)
                    x = oracle.sgemm(ta, tb, m, n, k, a, lda, b, ldb, c, ldc, acc)
                    y = ref.sgemm(ta, tb, m, n, k, a, lda, b, ldb, c, ldc, acc)
                    assert x.tobytes() == y.tobytes(), spec


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_underflowing_chains_end_at_negative_zero(oracle, ref, ta, tb):
    """An fma whose exact result is a nonzero negative value below half the least subnormal rounds to -0, and
    -0 + -0 = -0: nn-cpp's outputs are -0, depth cut or not, stored or added to a -0 C; the oracle agrees bit for
    bit, in both numerics modes (split pieces of -0 add to -0 too)."""
    for mode in (0, 1):
        oracle.set_numerics(mode)
        try:
            for m, n, k in UNDERFLOW_SHAPES:  # tile tails, depth cuts and split pieces of several lengths
                p = underflow_problem(ta, tb, m, n, k)
                for acc in (0, 1):
                    got = oracle.sgemm(ta, tb, m, n, k, p.a, p.lda, p.b, p.ldb, p.c, p.ldc, acc)[:m, :n]
                    assert np.all(got == 0) and np.all(np.signbit(got)), (mode, m, n, k, acc)
                    if mode == 0:
                        want = ref.sgemm(ta, tb, m, n, k, p.a, p.lda, p.b, p.ldb, p.c, p.ldc, acc)[:m, :n]
                        assert got.tobytes() == want.tobytes(), (m, n, k, acc)
        finally:
            oracle.set_numerics(0)


def test_oracle_ops_match_nncpp(oracle, ref):
    rng = np.random.default_rng(8)
    for _ in range(4):
        M, K, n = (int(v) for v in rng.integers(1, 80, 3))
        x, w, bias, g = (rng.uniform(-1, 1, s).astype(np.float32) for s in ((M, K), (n, K), (n,), (M, n)))
        assert oracle.linear_forward(x, w, bias).tobytes() == ref.linear_forward(x, w, bias).tobytes()
        got = oracle.linear_backward(g, x, w, dx_first=False, dw_first=False, db_first=False)
        for p, q in zip(got, ref.linear_backward(x, w, bias, g)):
            assert p.tobytes() == q.tobytes()
    for (N, Cin, H, W, Cout, kk, s, p_) in ((2, 3, 11, 9, 5, 3, 1, 1), (3, 1, 8, 8, 4, 2, 2, 0)):
        x = rng.uniform(-1, 1, (N, Cin, H, W)).astype(np.float32)
        w = rng.uniform(-1, 1, (Cout, Cin, kk, kk)).astype(np.float32)
        bias = rng.uniform(-1, 1, Cout).astype(np.float32)
        for relu in (0, 1):
            y, alive = oracle.conv2d_forward(x, w, bias, s, p_, relu)
            assert y.tobytes() == ref.conv2d_forward(x, w, bias, s, p_, relu).tobytes()
    for causal in (0, 1):
        q, k, v = (rng.standard_normal((2, 9, 12)).astype(np.float32) for _ in range(3))
        out, _ = oracle.attention_forward(q, k, v, 3, None, causal)
        assert out.tobytes() == ref.attention_forward(q, k, v, 3, None, causal).tobytes()
        x = rng.standard_normal((2, 3, 9, 9)).astype(np.float32)
        assert oracle.scaled_masked_softmax(x, 0.25, None, causal).tobytes() == \
            ref.scaled_masked_softmax(x, 0.25, None, causal).tobytes()


# ---------------------------------------------------------------- hand values from the reference's tests

def test_hand_values_matmul(oracle):
    """tests/test_tensor.cpp:365-383."""
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    got = oracle.sgemm(0, 0, 2, 2, 3, a, 3, b, 2, np.zeros((2, 2), np.float32), 2, 0)
    assert got.tolist() == [[58.0, 64.0], [139.0, 154.0]]
    ab = np.array([1, 0, 0, 1, 2, 0, 0, 2], np.float32).reshape(2, 2, 2)
    bb = np.ones((2, 2, 2), np.float32)
    c = oracle_matmul(oracle, ab, bb, 0, 0)
    assert c[0, 0, 0] == 1.0 and c[1, 0, 0] == 2.0


def test_hand_values_linear(oracle):
    """tests/test_nn.cpp:44-65: 1*3 + 2*4 + 0.5, and x W^T + b = 4.5, 9, 8.5, 16."""
    y = oracle.linear_forward(np.array([[3, 4]], np.float32), np.array([[1, 2]], np.float32), np.array([0.5], np.float32))
    assert y.tolist() == [[11.5]]
    w = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    y = oracle.linear_forward(np.array([[1, 0, 1], [0, 1, 2]], np.float32), w, np.array([0.5, -1.0], np.float32))
    assert y.tolist() == [[4.5, 9.0], [8.5, 16.0]]


def test_hand_values_conv(oracle):
    """tests/test_autograd.cpp:374-382: identity-diagonal 2x2 kernel over 1..9 gives 1+5 and 5+9."""
    x = np.arange(1, 10, dtype=np.float32).reshape(1, 1, 3, 3)
    w = np.array([1, 0, 0, 1], np.float32).reshape(1, 1, 2, 2)
    y, _ = oracle.conv2d_forward(x, w, np.zeros(1, np.float32), 1, 0, 0)
    assert y.shape == (1, 1, 2, 2) and y[0, 0, 0, 0] == 6.0 and y[0, 0, 1, 1] == 14.0


def test_hand_values_attention(oracle):
    """tests/test_transformer.cpp:149-176 (identity projections, one head, Dh = 2): softmax of x_i.x_j/sqrt(2)
    weights over the rows of x; and 269-276's fully masked row, which is exactly the mean of V."""
    x = np.array([1, 0, 0, 2], np.float32).reshape(1, 2, 2)
    out, _ = oracle.attention_forward(x, x, x, 1)
    s = np.float32(np.sqrt(2.0))
    for i in range(2):
        s0 = (x[0, i, 0] * x[0, 0, 0] + x[0, i, 1] * x[0, 0, 1]) / s
        s1 = (x[0, i, 0] * x[0, 1, 0] + x[0, i, 1] * x[0, 1, 1]) / s
        e0, e1 = np.exp(s0), np.exp(s1)
        for c in range(2):
            want = (e0 * x[0, 0, c] + e1 * x[0, 1, c]) / (e0 + e1)
            assert abs(out[0, i, c] - want) <= 1e-5 * abs(want) + 1e-7
    xs = synth.mt19937_uniform(3, 2 * 4 * 4).reshape(2, 4, 4)
    none = np.array([[0, 0, 0, 0], [1, 1, 1, 1]], np.float32)
    out, probs = oracle.attention_forward(xs, xs, xs, 2, none, False)
    assert np.all(np.isfinite(out))
    assert np.allclose(out[0], np.broadcast_to(xs[0].mean(axis=0), (4, 4)), rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- closed forms and identities

@pytest.mark.parametrize("ta,tb,acc", [(0, 0, 0), (1, 0, 1), (0, 1, 0), (1, 1, 1)])
def test_integer_products_are_exact(oracle, ta, tb, acc):
    """Small integers keep every partial sum exact (|sum| < 2^24), so any correct order gives the exact
    integer product: pins indexing, transposes, ld handling and the accumulate rule, depth cut included."""
    rng = np.random.default_rng(ta * 4 + tb * 2 + acc)
    for (m, n, k, pad) in ((7, 33, 17, 0), (64, 64, 1024, 3), (33, 5, 300, 1)):
        A = rng.integers(-4, 5, (m, k)).astype(np.float32)
        B = rng.integers(-4, 5, (k, n)).astype(np.float32)
        C0 = rng.integers(-100, 100, (m, n)).astype(np.float32)
        a = np.zeros(((k, m + pad) if ta else (m, k + pad)), np.float32)
        b = np.zeros(((n, k + pad) if tb else (k, n + pad)), np.float32)
        if ta:
            a[:, :m] = A.T
        else:
            a[:, :k] = A
        if tb:
            b[:, :k] = B.T
        else:
            b[:, :n] = B
        c = np.zeros((m, n + pad), np.float32)
        c[:, :n] = C0
        got = oracle.sgemm(ta, tb, m, n, k, a, a.shape[1], b, b.shape[1], c, n + pad, acc)
        exact = A.astype(np.int64) @ B.astype(np.int64) + (C0.astype(np.int64) if acc else 0)
        assert np.array_equal(got[:, :n].astype(np.int64), exact)
        assert np.all(got[:, n:] == 0.0)


def test_sgemm_within_north_star_bound_of_fp64(oracle):
    """|oracle - exact| <= 4 K 2^-24 sum|a||b| for random inputs (tolerance of BASELINE.json north_star)."""
    import golden_cases as gc
    for spec in ((0, 0, 65, 47, 600, 0, 1, 5), (1, 1, 64, 64, 1024, 1, 0, 6), (0, 1, 200, 100, 300, 1, 2, 7)):
        ta, tb, m, n, k, acc, pad, seed = spec
        a, lda, b, ldb, c, ldc = gc.sgemm_inputs(*spec)
        got = oracle.sgemm(ta, tb, m, n, k, a, lda, b, ldb, c, ldc, acc)
        exact, mag = oracle.sgemm_f64(ta, tb, m, n, k, a, lda, b, ldb, c, ldc, acc)
        assert np.all(np.abs(got[:, :n] - exact) <= 4 * k * 2.0 ** -24 * mag)


def test_sgemm_at_matches_full_product(oracle):
    import golden_cases as gc
    for spec in ((0, 0, 70, 90, 700, 1, 0, 9), (1, 0, 64, 64, 1024, 0, 2, 10), (0, 1, 33, 40, 20, 1, 1, 11)):
        ta, tb, m, n, k, acc, pad, seed = spec
        a, lda, b, ldb, c, ldc = gc.sgemm_inputs(*spec)
        full = oracle.sgemm(ta, tb, m, n, k, a, lda, b, ldb, c, ldc, acc)
        rows = np.arange(m).repeat(n)
        cols = np.tile(np.arange(n), m)
        got = oracle.sgemm_at(ta, tb, m, n, k, a, lda, b, ldb, acc, rows, cols, c[rows, cols])
        assert got.tobytes() == np.ascontiguousarray(full[:, :n]).reshape(-1).tobytes()


def test_depth_cut_predicate(oracle):
    """gemm.cpp:456-458 thresholds, at the cases of test_kernels.cpp:414."""
    assert oracle.depth_cut(64, 64, 1024) and oracle.depth_cut(40, 48, 589) and oracle.depth_cut(7, 300, 768)
    assert not oracle.depth_cut(64, 64, 511) and not oracle.depth_cut(300, 300, 512)
    assert not oracle.depth_cut(4096, 4096, 4096) and not oracle.depth_cut(64, 4096, 4096)
    assert not oracle.depth_cut(32, 9, 784)  # conv1 dW: m n k < 2^20


def test_im2col_definition_and_col2im_adjoint(oracle):
    """im2col equals the window definition; col2im is its adjoint: <im2col x, y> = <x, col2im y> (fp64)."""
    rng = np.random.default_rng(3)
    for (N, Cin, H, W, kk, s, p) in ((2, 3, 7, 6, 3, 2, 1), (1, 2, 5, 5, 4, 3, 3), (3, 1, 28, 28, 3, 1, 1)):
        x = rng.uniform(-1, 1, (N, Cin, H, W)).astype(np.float32)
        col = oracle.im2col(x, kk, kk, s, p)
        ho, wo = oracle.conv_out(H, W, kk, kk, s, p)
        xp = np.pad(x, ((0, 0), (0, 0), (p, p), (p, p)))
        for c in range(Cin):
            for i in range(kk):
                for j in range(kk):
                    win = xp[:, c, i:i + s * ho:s, j:j + s * wo:s][:, :ho, :wo].reshape(N, -1)
                    assert np.array_equal(col[:, (c * kk + i) * kk + j], win)
        y = rng.uniform(-1, 1, col.shape).astype(np.float32)
        back = oracle.col2im_add(y, np.zeros_like(x), kk, kk, s, p)
        lhs = float(np.sum(col.astype(np.float64) * y))
        rhs = float(np.sum(x.astype(np.float64) * back))
        assert abs(lhs - rhs) <= 1e-4 * (1 + abs(lhs))


def test_conv_close_to_fp64_direct_convolution(oracle):
    """test_autograd.cpp:420-448's direct-convolution reference, in fp64, with the north-star style bound."""
    rng = np.random.default_rng(4)
    for (N, Cin, H, W, Cout, kk, s, p) in ((7, 2, 9, 6, 3, 3, 2, 1), (3, 2, 33, 5, 2, 4, 3, 3), (2, 32, 14, 14, 8, 3, 1, 1)):
        x = rng.uniform(-1, 1, (N, Cin, H, W)).astype(np.float32)
        w = rng.uniform(-1, 1, (Cout, Cin, kk, kk)).astype(np.float32)
        b = rng.uniform(-1, 1, Cout).astype(np.float32)
        y, _ = oracle.conv2d_forward(x, w, b, s, p, 0)
        exact, mag = oracle.conv2d_f64(x, w, b, s, p)
        K = Cin * kk * kk
        assert np.all(np.abs(y - exact) <= 4 * (K + 1) * 2.0 ** -24 * mag)


def test_attention_close_to_fp64(oracle):
    rng = np.random.default_rng(5)
    for causal in (0, 1):
        q, k, v = (rng.standard_normal((2, 16, 32)).astype(np.float32) for _ in range(3))
        mask = np.ones((2, 16), np.float32)
        mask[1, 11:] = 0
        out, probs = oracle.attention_forward(q, k, v, 4, mask, causal)
        eo, ep = oracle.attention_f64(q, k, v, 4, mask, causal)
        assert np.allclose(probs, ep, rtol=1e-5, atol=1e-6)
        assert np.allclose(out, eo, rtol=1e-4, atol=1e-5)
        if causal:
            tri = np.triu(np.ones((16, 16), bool), 1)
            assert np.all(probs[:, :, tri] == 0.0)


def test_lane_sum_and_sum_axis0(oracle):
    """lane_sum's 8-lane order (ops.cpp:804-812) and Tensor::sum(0)'s row order differ from naive sums in
    their bits but not in value; integers make them exact."""
    p = np.arange(1, 100, dtype=np.float32)
    assert oracle.lane_sum(p) == np.float32(4950)
    x = np.arange(12, dtype=np.float32).reshape(4, 3)
    assert oracle.sum_axis0(x).tolist() == [18.0, 22.0, 26.0]
    v = synth.mt19937_uniform(1, 803)
    a = np.zeros(8, np.float32)
    for i in range(0, 800, 8):
        a += v[i:i + 8]
    t = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]))
    for i in range(800, 803):
        t = np.float32(t + v[i])
    assert oracle.lane_sum(v) == t


# ---------------------------------------------------------------- the softmax's exp

GOLDEN_DIR = os.path.join(HERE, "golden")
SOFTMAX_SRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "nn-cpp_amd", "src", "kernels",
                           "hip", "softmax_row.hpp")


def test_expf_table_is_its_definition():
    """kExp2Table of the GPU softmax's exp holds 2^(i/32) rounded to the nearest double, minus i << 47."""
    sys.path.insert(0, GOLDEN_DIR)
    from expf_table import exp2_table
    src = open(SOFTMAX_SRC).read()
    body = src[src.index("kExp2Table[32] = {"):]
    body = body[:body.index("};")]
    got = [int(v, 16) for v in re.findall(r"0x([0-9a-f]{16})ull", body)]
    assert got == exp2_table()


def test_expf_restatement_equals_glibc_expf(tmp_path):
    """The C form of the GPU softmax's exp (tests/golden/expf_glibc_check.c) returns the C library's expf bit for
    bit. Here on every 61st of the 2^32 inputs (70 million); the full scan (argument 1) also finds 0 differences."""
    exe = str(tmp_path / "expf_glibc_check")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", os.path.join(GOLDEN_DIR, "expf_glibc_check.c"), "-o", exe, "-lm"],
                   check=True)
    out = subprocess.run([exe, "61"], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0 and out.stdout.strip().endswith(" 0 differ"), out.stdout + out.stderr


# ---------------------------------------------------------------- max pooling (ops.cpp:1609-1705)

def test_golden_maxpool(oracle):
    """The oracle's forward and its scatter backward against nn-cpp's outputs (golden vectors), NaN, -inf windows,
    ties and overlapping windows included; NaN compares equal to NaN."""
    cases, gold = golden()
    for name, spec in cases.POOL_CASES:
        x, g, k, s = cases.pool_inputs(spec)
        y, arg = oracle.maxpool2d_forward(x, k, s)
        dx = oracle.maxpool2d_backward(g, arg, x.shape, k, s)
        want_y, want_dx = gold[f"pool/{name}/y"], gold[f"pool/{name}/dx"]
        assert np.array_equal(y, want_y, equal_nan=True) and y.tobytes() == want_y.tobytes(), name
        assert dx.tobytes() == want_dx.tobytes(), name


def test_maxpool_matches_nncpp(oracle, ref):
    """Against nn-cpp's compiled maxpool2d on larger random planes (config 3's 2 x 2 pooling and an overlapping
    window), with ties from quantised values."""
    for (N, C, H, W, k, s, seed) in ((4, 8, 28, 28, 2, 2, 71), (2, 3, 13, 11, 3, 2, 72), (1, 2, 10, 10, 4, 3, 73)):
        x, g = synth.uniform_operands(seed, [(N, C, H, W), (N, C, (H - k) // s + 1, (W - k) // s + 1)])
        x = (np.round(x * 8) / 8).astype(np.float32)
        y, arg = oracle.maxpool2d_forward(x, k, s)
        rc, ry, rdx = ref.maxpool2d(x, k, s, g)
        assert rc == 0
        assert y.tobytes() == ry.tobytes()
        assert oracle.maxpool2d_backward(g, arg, x.shape, k, s).tobytes() == rdx.tobytes()
    # the reference's shape errors: kernel larger than the plane, zero kernel or stride
    x = np.zeros((1, 1, 3, 3), np.float32)
    assert ref.maxpool2d(x, 4, 1)[0] == 2 and ref.maxpool2d(x, 0, 1)[0] == 2 and ref.maxpool2d(x, 2, 0)[0] == 2


def test_maxpool_hand_values(oracle):
    """Worked by hand: the first maximum of a window wins a tie; a window of -inf keeps -inf and offset 0, so its
    gradient lands on the plane's first element; NaN never wins; overlapping windows add in output order."""
    x = np.array([[[[1, 3, 3, 0],
                    [2, 3, 0, 5],
                    [-np.inf, -np.inf, np.nan, 4],
                    [-np.inf, -np.inf, 4, np.nan]]]], np.float32)
    y, arg = oracle.maxpool2d_forward(x, 2, 2)
    assert y.ravel().tolist() == [3, 5, -np.inf, 4]
    assert arg.ravel().tolist() == [1, 7, 0, 11]   # (0,1) wins the tie with (1,1); NaNs skipped
    g = np.array([10, 20, 30, 40], np.float32).reshape(1, 1, 2, 2)
    dx = oracle.maxpool2d_backward(g, arg, x.shape, 2, 2)
    want = np.zeros((4, 4), np.float32)
    want[0, 0], want[0, 1], want[1, 3], want[2, 3] = 30, 10, 20, 40
    assert dx.reshape(4, 4).tolist() == want.tolist()
    # overlapping 2 x 2 windows at stride 1 on a 1 x 3 ramp-down row pair: both windows pick x[0, 0] ... x[.., 1]
    x = np.array([[[[5, 4, 1], [0, 0, 0]]]], np.float32)
    y, arg = oracle.maxpool2d_forward(x, 2, 1)
    assert y.ravel().tolist() == [5, 4] and arg.ravel().tolist() == [0, 1]
    dx = oracle.maxpool2d_backward(np.array([[[[1.5, 2.5]]]], np.float32), arg, x.shape, 2, 1, dx=np.ones_like(x),
                                   first=False)
    assert dx.ravel().tolist() == [2.5, 3.5, 1, 1, 1, 1]


def test_softmax_backward_matches_nncpp(oracle, ref):
    """The oracle's scaled_masked_softmax backward against nn-cpp's backward rule (through its compiled library),
    with a key padding mask and causal rows; nn-cpp's leaf gradient starts zeroed, which gives the fresh rule's bits."""
    for (N, H, Tq, Tk, scale, masked, causal) in ((2, 3, 5, 7, 0.5, True, 0), (1, 2, 6, 6, 0.125, False, 1),
                                                  (2, 2, 9, 9, 1.0, True, 1)):
        x = synth.normal(120, (N, H, Tq, Tk))
        g = synth.normal(121, (N, H, Tq, Tk))
        pad = None
        if masked:
            pad = np.ones((N, Tk), np.float32)
            pad[0, -2:] = 0
        y = oracle.scaled_masked_softmax(x, np.float32(scale), pad, bool(causal))
        got = oracle.scaled_masked_softmax_backward(y, g, np.float32(scale), pad, bool(causal))
        want_y, want_dx = np.empty_like(x), np.empty_like(x)
        fp = lambda a: None if a is None else a.ctypes.data_as(__import__("ctypes").POINTER(__import__("ctypes").c_float))
        import ctypes as C
        rc = ref.lib.nnref_softmax_step(fp(x), C.c_size_t(N), C.c_size_t(H), C.c_size_t(Tq), C.c_size_t(Tk),
                                        C.c_float(scale), fp(pad), causal, fp(g), fp(want_y), fp(want_dx))
        assert rc == 0
        assert y.tobytes() == want_y.tobytes()
        assert got.tobytes() == want_dx.tobytes(), (N, H, Tq, Tk)


# ---------------------------------------------------------------- the split-depth numerics mode

@pytest.mark.parametrize("ta,tb,m,n,k,acc", [(0, 0, 64, 48, 300, 0), (1, 0, 33, 70, 256, 1), (0, 1, 100, 100, 784, 0),
                                             (1, 1, 16, 512, 513, 1), (0, 0, 512, 512, 600, 1), (1, 0, 256, 1024, 300, 0)])
def test_split_depth_oracle_is_nncpp_pieces_in_order(oracle, ref, ta, tb, m, n, k, acc):
    """In split mode a product with m n <= 2^18 and k >= 256 is cut as nn-cpp's depth cut is (gemm.cpp:466-484),
    with the split rule's piece depth: each slab of the depth is nn-cpp's own sgemm of that slab (a single chain
    from +0, the slab too short for nn-cpp to cut), the slabs are added in order, then stored or added to C.
    Checked against nn-cpp's compiled sgemm on each slab, summed here in float32, and against the fp64 bound."""
    from helpers import Problem
    p = Problem(ta, tb, m, n, k, 1, 5000 + m + n + k)
    oracle.set_numerics(1)
    try:
        pk = oracle.piece_depth(m, n, k)
        got = oracle.sgemm(ta, tb, m, n, k, p.a, p.lda, p.b, p.ldb, p.c, p.ldc, acc)
    finally:
        oracle.set_numerics(0)
    assert 0 < pk < k and not oracle.depth_cut(m, n, pk)
    opa = (p.a[:k, :m].T if ta else p.a[:m, :k])
    opb = (p.b[:n, :k].T if tb else p.b[:k, :n])
    total = None
    for k0 in range(0, k, pk):
        a_s = np.ascontiguousarray(opa[:, k0:k0 + pk])
        b_s = np.ascontiguousarray(opb[k0:k0 + pk, :])
        kk = a_s.shape[1]
        piece = ref.sgemm(0, 0, m, n, kk, a_s, kk, b_s, n, np.zeros((m, n), np.float32), n, 0)
        total = piece if total is None else (total + piece).astype(np.float32)
    want = (p.c[:m, :n] + total).astype(np.float32) if acc else total
    assert got[:m, :n].tobytes() == want.tobytes()
    exact, mag = oracle.sgemm_f64(ta, tb, m, n, k, p.a, p.lda, p.b, p.ldb, p.c, p.ldc, acc)
    assert np.all(np.abs(got[:m, :n].astype(np.float64) - exact) <= 4.0 * k * 2.0 ** -24 * mag)


def test_split_depth_rule(oracle):
    """The split rule: m n <= 2^18 and k >= 256; with T tiles of 64 x 16 and s = min(16, max(2, 4096 // T)), the
    pieces are ceil(k / s) rounded up to a multiple of 32 deep. Hand-computed cases; nn-cpp's own rule returns
    when the mode is reset."""
    oracle.set_numerics(1)
    try:
        # (m, n, k) -> piece depth, with the tile count T and piece count target s worked out by hand
        cases = {(512, 512, 512): 32,      # T = 8 * 32 = 256, s = 16, 32
                 (512, 512, 256): 32,      # s = 16, 16 -> 32
                 (64, 4096, 4096): 256,    # T = 1 * 256, s = 16, 256
                 (256, 512, 784): 64,      # T = 4 * 32 = 128, s = 16, ceil(784 / 16) = 49 -> 64
                 (256, 256, 512): 32,      # T = 64, s = 16, 32
                 (256, 10, 256): 32,       # T = 4, s = 16, 16 -> 32
                 (40, 48, 1100): 96,       # T = 3, s = 16, 69 -> 96
                 (16, 512, 513): 64,       # T = 32, s = 16, 33 -> 64
                 (1024, 256, 1000): 64,    # T = 16 * 16 = 256, s = 16, 63 -> 64
                 (512, 512, 2000): 128,    # s = 16, 125 -> 128
                 (65, 4000, 1000): 128,    # ragged: T = 2 * 250 = 500, s = 8, 125 -> 128
                 (1, 262144, 300): 160}    # T = 16384, s = 2 (the floor), 150 -> 160
        for (m, n, k), pk in cases.items():
            assert oracle.piece_depth(m, n, k) == pk, (m, n, k)
            assert oracle.depth_cut(m, n, k)
        assert oracle.piece_depth(2048, 2048, 16) == 0                    # m n > 2^18 (also at k 16)
        assert not oracle.depth_cut(512, 513, 4096)                       # m n > 2^18
        assert not oracle.depth_cut(512, 512, 255)                        # k < 256
    finally:
        oracle.set_numerics(0)
    assert not oracle.depth_cut(512, 512, 256) and oracle.depth_cut(40, 48, 1100)
    assert oracle.piece_depth(40, 48, 1100) == 128 and oracle.piece_depth(512, 512, 512) == 0


# ---------------------------------------------------------------- normalisation (ops.cpp:800-1078)

def test_golden_batchnorm_and_layernorm(oracle):
    """The restatements reproduce nn-cpp's outputs stored in the golden fixture: y, mean, var and the three
    gradients (fresh) of batchnorm with and without its folded ReLU, and layernorm's y and gradients."""
    gc, g = golden()
    for name, spec in gc.BATCHNORM_CASES:
        x, w, b, gr, relu = gc.batchnorm_inputs(spec)
        y, alive, mean, var, inv = oracle.batchnorm_forward(x, w, b, 1e-5, relu)
        dx, dw, db = oracle.batchnorm_backward(gr, x, alive, w, mean, inv)
        for key, val in (("y", y), ("mean", mean), ("var", var), ("dx", dx), ("dw", dw), ("db", db)):
            assert val.tobytes() == g[f"batchnorm/{name}/{key}"].tobytes(), (name, key)
    for name, spec in gc.LAYERNORM_CASES:
        x, gm, bt, gr = gc.layernorm_inputs(spec)
        y, mean, inv = oracle.layernorm_forward(x, gm, bt, 1e-5)
        dx, dg, db = oracle.layernorm_backward(gr, x, gm, mean, inv)
        for key, val in (("y", y), ("dx", dx), ("dgamma", dg), ("dbeta", db)):
            assert val.tobytes() == g[f"layernorm/{name}/{key}"].tobytes(), (name, key)


BN_SWEEP = [(4, 3, (5, 5)), (2, 5, (1, 1)), (3, 2, (17,)), (8, 4, (2, 3, 3)), (1, 1, ()), (64, 3, ()),
            (5, 2, (8,)), (2, 3, (2049,)), (300, 2, (1,))]


@pytest.mark.parametrize("shape", BN_SWEEP)
@pytest.mark.parametrize("relu", [0, 1])
def test_batchnorm_matches_nncpp(oracle, ref, shape, relu):
    """Against nn-cpp's compiled nn::batchnorm: rows with and without an eight-element tail, one element per row,
    many samples, rows longer than a staging chunk; the backward rule fresh and then added a second time."""
    N, Cc, sp = shape
    full = (N, Cc) + tuple(sp)
    rng = np.random.default_rng(N * 31 + Cc + relu)
    x = (rng.uniform(-3, 5, full)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, Cc).astype(np.float32)
    b = rng.uniform(-1, 1, Cc).astype(np.float32)
    g = rng.normal(size=full).astype(np.float32)
    y, alive, mean, var, inv = oracle.batchnorm_forward(x, w, b, 1e-5, relu)
    rc, yr, mr, vr, (dxr, dwr, dbr) = ref.batchnorm(x, w, b, 1e-5, relu, g=g)
    assert rc == 0
    assert y.tobytes() == yr.tobytes() and mean.tobytes() == mr.tobytes() and var.tobytes() == vr.tobytes()
    dx, dw, db = oracle.batchnorm_backward(g, x, alive, w, mean, inv)
    assert (dx.tobytes(), dw.tobytes(), db.tobytes()) == (dxr.tobytes(), dwr.tobytes(), dbr.tobytes())
    rc, _, _, _, (dx2r, dw2r, db2r) = ref.batchnorm(x, w, b, 1e-5, relu, g=g, repeats=2)
    dx2, dw2, db2 = oracle.batchnorm_backward(g, x, alive, w, mean, inv, dx, False, dw, False, db, False)
    assert (dx2.tobytes(), dw2.tobytes(), db2.tobytes()) == (dx2r.tobytes(), dw2r.tobytes(), db2r.tobytes())


@pytest.mark.parametrize("shape", [(5, 4), (3, 7, 64), (2, 1), (9, 33), (40, 30, 16), (2, 515)])
def test_layernorm_matches_nncpp(oracle, ref, shape):
    D = shape[-1]
    rng = np.random.default_rng(sum(shape))
    x = rng.uniform(-2, 3, shape).astype(np.float32)
    gm = rng.uniform(0.5, 1.5, D).astype(np.float32)
    bt = rng.uniform(-1, 1, D).astype(np.float32)
    g = rng.normal(size=shape).astype(np.float32)
    y, mean, inv = oracle.layernorm_forward(x, gm, bt, 1e-5)
    rc, yr, (dxr, dgr, dbr) = ref.layernorm(x.reshape(-1, D), gm, bt, 1e-5, g=g.reshape(-1, D))
    assert rc == 0 and y.tobytes() == yr.reshape(shape).tobytes()
    dx, dg, db = oracle.layernorm_backward(g, x, gm, mean, inv)
    assert (dx.tobytes(), dg.tobytes(), db.tobytes()) == (dxr.reshape(shape).tobytes(), dgr.tobytes(), dbr.tobytes())
    rc, _, (dx2r, dg2r, db2r) = ref.layernorm(x.reshape(-1, D), gm, bt, 1e-5, g=g.reshape(-1, D), repeats=2)
    dx2, dg2, db2 = oracle.layernorm_backward(g, x, gm, mean, inv, dx, False, dg, False, db, False)
    assert (dx2.tobytes(), dg2.tobytes(), db2.tobytes()) == (dx2r.reshape(shape).tobytes(), dg2r.tobytes(),
                                                             db2r.tobytes())


def test_batchnorm_hand_values_and_fp64(oracle):
    """Hand values (test_nn.cpp:527-537's batches): {0, 2} has mean 1 and biased variance 1, so with eps 0 the
    output is exactly -1, 1; {4, 4} has mean 4 and variance 0. Then against the fp64 normalisation: every channel of
    the output has mean 0 and variance 1 (test_nn.cpp:341-354's criterion), and y = xhat * w + b within a few ulps;
    the gradients satisfy the identities of the exact backward: sum(dx) = 0 and sum(dx * xhat) = 0 per channel,
    db = sum(g), dw = sum(g * xhat)."""
    y, _, mean, var, _ = oracle.batchnorm_forward(np.array([[0], [2]], np.float32), np.ones(1, np.float32),
                                                  np.zeros(1, np.float32), 0.0)
    assert y.ravel().tolist() == [-1.0, 1.0] and mean.tolist() == [1.0] and var.tolist() == [1.0]
    _, _, mean, var, _ = oracle.batchnorm_forward(np.array([[4], [4]], np.float32), np.ones(1, np.float32),
                                                  np.zeros(1, np.float32), 1e-5)
    assert mean.tolist() == [4.0] and var.tolist() == [0.0]
    rng = np.random.default_rng(5)
    x = rng.uniform(-3, 5, (8, 3, 5, 5)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 3).astype(np.float32)
    b = rng.uniform(-1, 1, 3).astype(np.float32)
    g = rng.normal(size=x.shape).astype(np.float32)
    y, _, mean, var, inv = oracle.batchnorm_forward(x, w, b, 1e-5)
    xhat = oracle.batchnorm_f64(x, 1e-5)
    ref64 = xhat * w[None, :, None, None] + b[None, :, None, None]
    assert np.max(np.abs(y - ref64)) < 1e-5
    yn = (y - b[None, :, None, None]) / w[None, :, None, None]
    assert np.all(np.abs(yn.mean(axis=(0, 2, 3))) < 1e-3) and np.all(np.abs(yn.var(axis=(0, 2, 3)) - 1) < 1e-3)
    dx, dw, db = oracle.batchnorm_backward(g, x, None, w, mean, inv)
    assert np.max(np.abs(dx.astype(np.float64).sum(axis=(0, 2, 3)))) < 1e-3
    assert np.max(np.abs((dx * xhat).sum(axis=(0, 2, 3)))) < 1e-3
    assert np.allclose(db, g.astype(np.float64).sum(axis=(0, 2, 3)), atol=1e-4)
    assert np.allclose(dw, (g * xhat).sum(axis=(0, 2, 3)), atol=1e-3)


def test_layernorm_hand_values_and_fp64(oracle):
    """test_transformer.cpp:64-80: the row 1, 2, 3, 4 comes out with mean 0 and variance 1, a constant row comes out
    0, and equal rows come out equal whatever the leading shape; fp64 normalisation within a few ulps; dbeta is the
    column sum of g and dgamma the column sum of g * xhat."""
    ones, zeros = np.ones(4, np.float32), np.zeros(4, np.float32)
    y, _, _ = oracle.layernorm_forward(np.array([[1, 2, 3, 4]], np.float32), ones, zeros, 1e-5)
    assert abs(y.mean()) < 1e-4 and abs(((y - y.mean()) ** 2).mean() - 1) < 1e-4
    c, _, _ = oracle.layernorm_forward(np.full((1, 4), 3, np.float32), ones, zeros, 1e-5)
    assert np.all(c == 0)
    rows, _, _ = oracle.layernorm_forward(np.tile(np.array([1, 2, 3, 4], np.float32), (2, 3, 1)), ones, zeros, 1e-5)
    assert all(r.tobytes() == y.ravel().tobytes() for r in rows.reshape(-1, 4))
    rng = np.random.default_rng(6)
    x = rng.uniform(-2, 3, (40, 30, 16)).astype(np.float32)
    gm = rng.uniform(0.5, 1.5, 16).astype(np.float32)
    bt = rng.uniform(-1, 1, 16).astype(np.float32)
    g = rng.normal(size=x.shape).astype(np.float32)
    y, mean, inv = oracle.layernorm_forward(x, gm, bt, 1e-5)
    xhat = oracle.layernorm_f64(x, 1e-5)
    assert np.max(np.abs(y - (xhat * gm + bt))) < 1e-5
    dx, dg, db = oracle.layernorm_backward(g, x, gm, mean, inv)
    assert np.allclose(db, g.reshape(-1, 16).astype(np.float64).sum(0), atol=1e-3)
    assert np.allclose(dg, (g * xhat).reshape(-1, 16).sum(0), atol=1e-3)
    assert np.max(np.abs(dx.astype(np.float64).sum(-1))) < 1e-4


# ---------------------------------------------------------------- element-wise: GELU, embedding

def _gelu_inputs(seed=0):
    rng = np.random.default_rng(seed)
    x = np.concatenate([rng.normal(size=50000).astype(np.float32) * 3,
                        np.linspace(-12, 12, 20001).astype(np.float32),  # both sides of the +-9 clamp of 2z
                        np.array([0, -0.0, 1e-30, -1e-30, 1e4, -1e4, np.inf, -np.inf, np.nan], np.float32)])
    return x, rng.normal(size=x.size).astype(np.float32)


def _bits_nan_equal(a, b):
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a.view(np.uint32)[~na], b.view(np.uint32)[~nb])


def test_gelu_matches_nncpp(oracle, ref):
    """Against nn-cpp's compiled nn::gelu (its AVX2 eight-lane tanh for whole groups of eight and the scalar form for
    the tail): forward, the saved tanh feeding the backward rule, fresh and added gradients."""
    x, g = _gelu_inputs()
    y, th = oracle.gelu_forward(x)
    rc, yr, dxr = ref.gelu(x, g)
    assert rc == 0 and _bits_nan_equal(y, yr)
    dx = oracle.gelu_backward(x, th, g)
    assert _bits_nan_equal(dx, dxr)
    rc, _, dx2r = ref.gelu(x, g, repeats=2)
    assert _bits_nan_equal(oracle.gelu_backward(x, th, g, dx, False), dx2r)


def test_gelu_against_the_closed_form(oracle):
    """y = x/2 (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) in fp64 within 2e-6 of |y| + 1e-6 (the tanh is computed as
    (e^2z - 1)/(e^2z + 1), which loses relative precision near 0); tanh(0) = 0, tanh(+-20) = +-1 exactly, NaN stays NaN;
    the derivative against a central difference of the fp64 form."""
    x, g = _gelu_inputs(1)
    y, th = oracle.gelu_forward(x)
    fin = np.isfinite(x) & (np.abs(x) < 100)
    xd = x[fin].astype(np.float64)
    want = 0.5 * xd * (1 + np.tanh(np.sqrt(2 / np.pi) * (xd + 0.044715 * xd ** 3)))
    assert np.all(np.abs(y[fin] - want) <= 2e-6 * np.abs(want) + 1e-6)
    assert oracle.lib.oracle_tanh_one(0.0) == 0.0 and oracle.lib.oracle_tanh_one(20.0) == 1.0
    assert oracle.lib.oracle_tanh_one(-20.0) == -1.0 and np.isnan(oracle.lib.oracle_tanh_one(float("nan")))
    f = lambda v: 0.5 * v * (1 + np.tanh(np.sqrt(2 / np.pi) * (v + 0.044715 * v ** 3)))
    xs = np.linspace(-6, 6, 1001).astype(np.float32)
    _, ths = oracle.gelu_forward(xs)
    d = oracle.gelu_backward(xs, ths, np.ones_like(xs))
    h = 1e-5
    num = (f(xs.astype(np.float64) + h) - f(xs.astype(np.float64) - h)) / (2 * h)
    assert np.max(np.abs(d - num)) < 1e-5


def test_embedding_matches_nncpp(oracle, ref):
    """Rows gathered; the gradient table gets the output rows added in token order (repeated ids included), fresh
    and added; ids that nn-cpp rejects (fractional, negative, past the table) throw TensorShapeError there."""
    rng = np.random.default_rng(2)
    w = rng.normal(size=(64, 32)).astype(np.float32)
    ids = rng.integers(0, 64, 500).astype(np.float32)
    g = rng.normal(size=(500, 32)).astype(np.float32)
    rc, y, dwr = ref.embedding(w, ids, g)
    assert rc == 0 and np.array_equal(y, w[ids.astype(int)])
    rows = ids.astype(np.int32)
    dw = oracle.embedding_backward(g, rows, 64, 32)
    assert dw.tobytes() == dwr.tobytes()
    # hand values: two tokens on row 3 add in order, untouched rows are +0
    small = oracle.embedding_backward(np.array([[1.0], [2.0], [-1.0]], np.float32), np.array([3, 3, 0], np.int32), 5, 1)
    assert small.ravel().tolist() == [-1.0, 0.0, 0.0, 3.0, 0.0]
    rc, _, dw2r = ref.embedding(w, ids, g, repeats=2)
    assert oracle.embedding_backward(g, rows, 64, 32, dw, False).tobytes() == dw2r.tobytes()
    for bad in (1.5, 64.0, -1.0):
        assert ref.embedding(w, np.array([bad], np.float32))[0] == 2


# ---------------------------------------------------------------- transformer_tiny workload definition

def test_transformer_tiny_layout_matches_nncpp(ref):
    """The GPU harness's parameter list (nnh/workloads.py, nn-cpp_amd/src/bench/workloads.cpp) is nn-cpp's
    Transformer{vocab 64, dim 64, heads 4, layers 2, max_len 64}: the same shapes in the same order, and the gammas
    that reseed_parameters keeps at one are exactly the parameters that start at one."""
    from nnh import workloads as wl
    w = wl.by_name("transformer_tiny")
    layout = ref.transformer_tiny_layout()
    assert [s for s, _ in layout] == [tuple(s) for s in w.shapes]
    assert [i for i, (s, ones) in enumerate(layout) if ones and len(s) < 2] == list(w.ones)


def test_transformer_tiny_ids_and_reference_step(ref):
    """make_transformer_tiny's ids are std::uniform_int_distribution<int>(0, 63) over std::mt19937(seed + 1): here the
    top six bits of each draw, every id a whole number in [0, 64) with all 64 present; nn-cpp's own training step on
    them runs, is deterministic, and gives finite logits and gradients."""
    from nnh import workloads as wl
    w = wl.by_name("transformer_tiny")
    params, x, g = wl.inputs(w, 1)
    assert x.shape == (16, 64) and np.all(x == np.floor(x)) and x.min() == 0 and x.max() == 63
    assert len(np.unique(x)) == 64
    assert all(np.all(params[i] == 1) for i in w.ones)
    runs = [wl.run_step(ref.lib.nnref_time_workload_step, w, params, x, g, 0, 1, want_grads=True) for _ in range(2)]
    for rc, _, _, logits, grads in runs:
        assert rc == 0 and np.all(np.isfinite(logits)) and all(np.all(np.isfinite(a)) for a in grads)
    assert runs[0][3].tobytes() == runs[1][3].tobytes()
    assert all(a.tobytes() == b.tobytes() for a, b in zip(runs[0][4], runs[1][4]))

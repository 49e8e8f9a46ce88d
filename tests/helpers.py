"""Problem builders shared by the tests (the shape of tests/test_kernels.cpp:51-86)."""
import numpy as np

from nnh import synth

SENTINEL = np.float32(1e30)


class Problem:
    """op(A) m x k, op(B) k x n, C m x n, stored per the transpose flags with `pad` extra columns of
    sentinel in every leading dimension, values from the reference's seeded uniform stream."""

    def __init__(self, ta, tb, m, n, k, pad, seed, lo=-1.0, hi=1.0):
        self.ta, self.tb, self.m, self.n, self.k = ta, tb, m, n, k
        a_rows, a_cols = (k, m) if ta else (m, k)
        b_rows, b_cols = (n, k) if tb else (k, n)
        self.lda, self.ldb, self.ldc = a_cols + pad, b_cols + pad, n + pad
        vals = synth.mt19937_uniform(seed, a_rows * a_cols + b_rows * b_cols + m * n, lo, hi)
        self.a = self._fill(vals[: a_rows * a_cols], a_rows, a_cols, self.lda)
        o = a_rows * a_cols
        self.b = self._fill(vals[o: o + b_rows * b_cols], b_rows, b_cols, self.ldb)
        o += b_rows * b_cols
        self.c = self._fill(vals[o:], m, n, self.ldc)

    @staticmethod
    def _fill(v, rows, cols, ld):
        out = np.full((max(rows, 1), max(ld, 1)), SENTINEL, np.float32)
        if rows and cols:
            out[:rows, :cols] = v.reshape(rows, cols)
        return np.ascontiguousarray(out)

    def args(self):
        return (self.ta, self.tb, self.m, self.n, self.k)


def underflow_problem(ta, tb, m, n, k, pad=1):
    """Every product is -2^-160: it rounds to -0, so each chain from +0 turns into -0 at its first step and stays
    there, and a sum of -0 pieces is -0. A depth step that adds +0 (a zero-padded tail) turns it into +0."""
    p = Problem(ta, tb, m, n, k, pad, 1)
    p.a[...] = np.float32(-(2.0 ** -80))
    p.b[...] = np.float32(2.0 ** -80)
    p.c[...] = np.float32(-0.0)
    return p


# Depths past tile sizes (16, 32), depth cuts with short last pieces, and split-mode shapes
UNDERFLOW_SHAPES = [(7, 9, 17), (33, 40, 100), (65, 129, 257), (40, 48, 1100), (64, 64, 1024), (5, 9, 1100),
                    (256, 10, 300), (100, 100, 777)]


def gpu_sgemm(p, acc, config=-1, c=None, batch=None, epilogue=None):
    """Runs the product's sgemm on copies of p's buffers; returns the whole C buffer."""
    import torch

    import nnh
    dev = torch.device("cuda:0")
    a = torch.from_numpy(p.a).to(dev)
    b = torch.from_numpy(p.b).to(dev)
    cc = torch.from_numpy(np.array(p.c if c is None else c, copy=True)).to(dev)
    if config == -1 and batch is None and epilogue is None:
        nnh.sgemm(p.ta, p.tb, p.m, p.n, p.k, a, p.lda, b, p.ldb, cc, p.ldc, acc)
    else:
        nnh.sgemm_batched(p.ta, p.tb, p.m, p.n, p.k, a, p.lda, b, p.ldb, cc, p.ldc, acc, batch, epilogue, config)
    torch.cuda.synchronize()
    return cc.cpu().numpy()


def oracle_sgemm(oracle, p, acc, c=None):
    return oracle.sgemm(p.ta, p.tb, p.m, p.n, p.k, p.a, p.lda, p.b, p.ldb, p.c if c is None else c, p.ldc, acc)


def bits_equal(x, y):
    return x.shape == y.shape and x.tobytes() == y.tobytes()


def assert_same(got, want, what, nan_equal=False):
    """Bit-for-bit equality of two arrays (with nan_equal, any NaN matches any NaN). The comparison is made
    before the assert, so a failure reports the first difference instead of a diff of the raw bytes."""
    assert got.shape == want.shape, (what, got.shape, want.shape)
    if got.dtype == np.float32 and want.dtype == np.float32:
        diff = got.view(np.uint32) != want.view(np.uint32)
        if nan_equal:
            diff &= ~(np.isnan(got) & np.isnan(want))
    else:
        diff = got != want
    bad = np.nonzero(diff)
    ok = len(bad[0]) == 0
    if not ok:
        idx = tuple(int(v[0]) for v in bad)
        msg = f"{what}: {len(bad[0])} differ, first at {idx}: got {got[idx]!r} want {want[idx]!r}"
    assert ok, msg


def first_diff(x, y):
    d = np.nonzero(x.view(np.uint32) != y.view(np.uint32))
    if len(d[0]) == 0:
        return "identical"
    idx = tuple(int(v[0]) for v in d)
    return f"{len(d[0])} differ, first at {idx}: got {x[idx]!r} want {y[idx]!r}"


def within_fp64_bound(got, p, acc, oracle, c_in=None):
    """|got - exact| <= 4 K 2^-24 sum|a||b| (+|c| when accumulating), against fp64."""
    exact, mag = oracle.sgemm_f64(p.ta, p.tb, p.m, p.n, p.k, p.a, p.lda, p.b, p.ldb,
                                  p.c if c_in is None else c_in, p.ldc, acc)
    g = got[: p.m, : p.n].astype(np.float64)
    bound = 4.0 * max(p.k, 1) * 2.0 ** -24 * mag
    fin = np.isfinite(exact)
    return bool(np.all(np.abs(g[fin] - exact[fin]) <= bound[fin]))

"""The row softmax's division (div_by_row_sum in nn-cpp_amd/src/kernels/hip/softmax_row.hpp) against IEEE float
division, the reference's `o[j] /= sum` (src/autograd/ops.cpp:1203).

The GPU computes q = (double)p * (1 / (double)s), rounds q to float, and takes the float division only for
positive quotients below 2^-125. numpy's float64 product, float64 reciprocal and float64 -> float32 conversion are
the same IEEE operations (round to nearest even, subnormals kept) as the GPU's v_mul_f64, the f64 division and
v_cvt_f32_f64, so this checks the method itself. The operands are those a softmax row can produce (0 <= p <= s,
s up to a few thousand) and the hardest ones for the method: quotients within a few double ulps of a float
midpoint, subnormal quotients that are exactly midpoints, divisors that are not powers of two.
"""
import numpy as np

F32 = np.float32


def method(p, s):
    p = np.asarray(p, np.float32)
    s = np.asarray(s, np.float32)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore", under="ignore"):
        rinv = 1.0 / s.astype(np.float64)
        q = p.astype(np.float64) * rinv
        fallback = (q > 0.0) & (q < 2.0 ** -125)
        return np.where(fallback, p / s, q.astype(np.float32))


def ieee(p, s):
    with np.errstate(divide="ignore", invalid="ignore", over="ignore", under="ignore"):
        return np.asarray(p, np.float32) / np.asarray(s, np.float32)


def check(p, s, what):
    got, want = method(p, s), ieee(p, s)
    gb, wb = got.view(np.uint32), want.view(np.uint32)
    bad = (gb != wb) & ~(np.isnan(got) & np.isnan(want))
    assert not bad.any(), (what, int(bad.sum()), p[bad][:4], s[bad][:4], got[bad][:4], want[bad][:4])


def random_floats(rng, n, lo_bits, hi_bits):
    return rng.integers(lo_bits, hi_bits, n, dtype=np.uint64).astype(np.uint32).view(np.float32)


def test_random_softmax_operands():
    rng = np.random.default_rng(7)
    n = 4_000_000
    s = random_floats(rng, n, 0x3f800000, 0x45800000)  # sums in [1, 4096)
    p = random_floats(rng, n, 0x00000001, 0x3f800001)  # exponentials in (0, 1], subnormals included
    check(p, s, "random p in (0, 1], s in [1, 4096)")
    s2 = random_floats(rng, n, 0x00000001, 0x3f800000)  # degenerate rows: sums below 1 (all keys masked)
    p2 = (s2 * rng.random(n, dtype=np.float32)).astype(np.float32)
    check(p2, s2, "p <= s < 1")


def test_quotients_next_to_midpoints():
    """p = s * m rounded, for m a midpoint between consecutive floats: the quotient lies within an ulp of p of the
    midpoint, the case where an approximate quotient could round the wrong way."""
    rng = np.random.default_rng(11)
    n = 2_000_000
    s = random_floats(rng, n, 0x3f800000, 0x45800000)
    lo = random_floats(rng, n, 0x20000000, 0x3f800000).astype(np.float64)  # m in [2^-63, 1)
    m = lo + np.spacing(lo.astype(np.float32)).astype(np.float64) / 2
    p = (s.astype(np.float64) * m).astype(np.float32)
    for dp in (-2, -1, 0, 1, 2):
        pp = (p.view(np.uint32).astype(np.int64) + dp).astype(np.uint32).view(np.float32)
        keep = (pp > 0) & (pp <= s)
        check(pp[keep], s[keep], ("near midpoints", dp))


def test_small_integer_sums_and_subnormal_quotients():
    """s = small integers times powers of two (rows with a few keys at the maximum) against every p = k 2^-149 for
    k < 2^14 and a spread of normal p: includes subnormal quotients that are exactly midpoints (p = 6 m)."""
    ints = np.arange(1, 300, dtype=np.float32)
    s = np.concatenate([ints, ints * 2, ints * 1024, ints / 4]).astype(np.float32)
    k = np.arange(1, 1 << 14, dtype=np.uint32).view(np.float32)  # k * 2^-149
    pp, ss = np.meshgrid(k, s)
    check(pp.ravel(), ss.ravel(), "subnormal p")
    rng = np.random.default_rng(5)
    pn = random_floats(rng, 20000, 0x00800000, 0x3f800001)
    pp, ss = np.meshgrid(pn, s)
    check(pp.ravel(), ss.ravel(), "normal p")


def test_special_operands():
    inf, nan = F32(np.inf), F32(np.nan)
    p = np.array([0, 0, 0, 1, nan, 0, 1, 0.5, 2 ** -149, 2 ** -149, 1], np.float32)
    s = np.array([1, 0, nan, nan, 3, 2 ** -149, 2 ** -149, 0.5, 6, 0.75, inf], np.float32)
    check(p, s, "special operands")
    assert method(np.float32(0), np.float32(5)).view(np.uint32) == 0  # +0, as 0 / s

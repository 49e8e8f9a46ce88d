"""Parity of nnh_sgemm (the replacement of nn::kernels::sgemm) with nn-cpp, on the GPU.

Mirrors tests/test_kernels.cpp of the reference (sizes x flags x accumulate, block boundaries, zero sizes,
leading-dimension padding with sentinels, Inf/NaN, determinism, the depth cut), but the bar is higher:
every output must be BIT-IDENTICAL to the oracle, which restates nn-cpp's NN_NATIVE arithmetic and is
itself pinned bit for bit to nn-cpp's compiled sources (tests/test_oracle.py). Full BASELINE sizes are
checked on sampled elements (the oracle recomputes each sampled element's whole depth chain).
"""
import numpy as np
import pytest

from helpers import (SENTINEL, UNDERFLOW_SHAPES, Problem, assert_same, bits_equal, first_diff, gpu_sgemm,
                     oracle_sgemm, underflow_problem, within_fp64_bound)
from nnh import synth

pytestmark = pytest.mark.gpu


def check(oracle, p, acc, config=-1):
    got = gpu_sgemm(p, acc, config)
    want = oracle_sgemm(oracle, p, acc)
    assert bits_equal(got, want), f"ta={p.ta} tb={p.tb} m={p.m} n={p.n} k={p.k} acc={acc}: {first_diff(got, want)}"
    return got


def test_sizes_and_flags(gpu, oracle):
    """test_kernels.cpp:293-331: sizes {1,7,33,257}^3 x trans_a x trans_b x accumulate."""
    sizes = (1, 7, 33, 257)
    seed = 4000
    for ta in (0, 1):
        for tb in (0, 1):
            for acc in (0, 1):
                for m in sizes:
                    for n in sizes:
                        for k in sizes:
                            check(oracle, Problem(ta, tb, m, n, k, 0, seed), acc)
                            seed += 1


def test_block_boundaries(gpu, oracle):
    """Past each of the reference's block sizes (kMC=96, kKC=256, kNC=1024; test_kernels.cpp:169-178) and
    past each of this kernel's tile sizes (64/128/256 rows, 128 columns, 16/32 deep)."""
    cases = [(96 + 5, 7, 33), (7, 33, 256 + 5), (7, 1024 + 5, 33), (7, 1024 + 5, 256 + 5),
             (257, 129, 17), (129, 129, 33), (255, 127, 31), (65, 300, 64), (300, 200, 100), (512, 384, 48)]
    seed = 1000
    for ta in (0, 1):
        for tb in (0, 1):
            for acc in (0, 1):
                for m, n, k in cases:
                    check(oracle, Problem(ta, tb, m, n, k, 0, seed), acc)
                    seed += 1


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_underflowing_chains_keep_negative_zero(gpu, oracle, ta, tb):
    """Chains whose every product rounds to -0 end at -0 in nn-cpp (and -0 + -0 = -0 when accumulating): the
    steps past the depth in a kernel's last depth tile or last piece must leave -0 alone, in every tile
    configuration."""
    import nnh
    for m, n, k in UNDERFLOW_SHAPES:
        p = underflow_problem(ta, tb, m, n, k)
        for acc in (0, 1):
            want = oracle_sgemm(oracle, p, acc)
            assert np.all(np.signbit(want[:m, :n]))
            got = gpu_sgemm(p, acc)
            assert bits_equal(got, want), ((m, n, k), acc, first_diff(got, want))
    p = underflow_problem(ta, tb, 40, 48, 100)
    want = oracle_sgemm(oracle, p, 0)
    for cfg in range(len(nnh.gemm_configs())):
        got = gpu_sgemm(p, 0, config=cfg)
        assert bits_equal(got, want), (cfg, first_diff(got, want))


def test_zero_size_dimensions(gpu):
    """test_kernels.cpp:180-201: m or n == 0 touches nothing; k == 0 zero-fills, or leaves C when
    accumulating; nothing outside m x n is written."""
    import torch

    import nnh
    for m, n, k in ((0, 5, 4), (3, 0, 4), (3, 5, 0)):
        for acc in (0, 1):
            ldc = 6
            a = torch.ones(16, device="cuda")
            b = torch.ones(32, device="cuda")
            c = np.full((4, ldc), SENTINEL, np.float32)
            c[:m, :n] = 2.0
            cd = torch.from_numpy(c).cuda()
            nnh.sgemm(0, 0, m, n, k, a, k if k else 1, b, n if n else 1, cd, ldc, acc)
            got = cd.cpu().numpy()
            want = np.full((4, ldc), SENTINEL, np.float32)
            want[:m, :n] = 2.0 if acc else 0.0
            assert bits_equal(got, want), (m, n, k, acc)


def test_leading_dimensions_wider_than_width(gpu, oracle):
    """test_kernels.cpp:203-209 (sentinel padding stays untouched, bitwise), plus larger and odd pads that
    break 16-byte alignment of rows."""
    seed = 2000
    for ta in (0, 1):
        for tb in (0, 1):
            for acc in (0, 1):
                for (m, n, k, pad) in ((7, 33, 33, 3), (200, 300, 100, 5), (128, 128, 64, 1), (256, 256, 256, 4)):
                    check(oracle, Problem(ta, tb, m, n, k, pad, seed), acc)
                    seed += 1


def test_inf_and_nan_propagate(gpu, oracle):
    """test_kernels.cpp:211-231: op(A)(2,0) = +Inf, row 0 of op(B) cycles +1, -1, 0 (so row 2 of C holds
    +Inf, -Inf and NaN), op(B)(5,3) = NaN (column 3 of C is NaN)."""
    seed = 3000
    for ta in (0, 1):
        for tb in (0, 1):
            for acc in (0, 1):
                p = Problem(ta, tb, 7, 33, 17, 0, seed)
                seed += 1
                if ta:
                    p.a[0, 2] = np.inf
                else:
                    p.a[2, 0] = np.inf
                for j in range(p.n):
                    v = 1.0 if j % 3 == 0 else (-1.0 if j % 3 == 1 else 0.0)
                    if tb:
                        p.b[j, 0] = v
                    else:
                        p.b[0, j] = v
                if tb:
                    p.b[3, 5] = np.nan
                else:
                    p.b[5, 3] = np.nan
                got = check(oracle, p, acc)
                assert np.isnan(got[2, 2]) and np.isposinf(got[2, 0]) and np.isneginf(got[2, 1])
                assert np.all(np.isnan(got[:, 3]))


def test_deterministic_repeat(gpu):
    """test_kernels.cpp:333-341, and repeated large launches: bitwise identical run to run."""
    for (ta, tb, m, n, k, pad, seed) in ((0, 1, 101, 75, 300, 2, 5000), (0, 0, 1024, 1024, 1024, 0, 5001),
                                         (1, 0, 300, 1000, 700, 3, 5002)):
        p = Problem(ta, tb, m, n, k, pad, seed)
        for acc in (0, 1):
            first = gpu_sgemm(p, acc)
            for _ in range(2):
                assert bits_equal(gpu_sgemm(p, acc), first)


def test_depth_cut(gpu, oracle):
    """test_kernels.cpp:406-435: small m x n with a long depth is cut into 128-deep pieces summed in order;
    the shapes just under the thresholds take the ordinary path."""
    cases = [(64, 64, 1024), (40, 48, 2 * 256 + 77), (7, 300, 3 * 256), (64, 64, 2 * 256 - 1), (300, 300, 512)]
    seed = 30000
    for ta in (0, 1):
        for tb in (0, 1):
            for acc in (0, 1):
                for m, n, k in cases:
                    check(oracle, Problem(ta, tb, m, n, k, 3, seed), acc)
                    seed += 1


def _chain4_config():
    import nnh
    return next(i for i, nm in enumerate(nnh.gemm_configs()) if nm.startswith("mfma chain 16x16x4"))


@pytest.mark.parametrize("force_chain", [0, 1])
def test_accumulate_adds_old_c_after_first_depth_block(gpu, oracle, force_chain):
    """With accumulate, nn-cpp adds the old C after the first 256 depth steps (Store::kAdd, then
    kContinue): exercised at depths around 256 and 512, with and without the depth cut, aligned and padded rows;
    force_chain runs the products that are not cut on the whole-depth 16x16x4 chain kernel (old C added between two
    of its 128-deep chunks)."""
    cfg = _chain4_config() if force_chain else -1
    seed = 40000
    for k in (1, 15, 255, 256, 257, 300, 511, 512, 513, 1000):
        for (m, n) in ((129, 129), (300, 300)):
            for ta, tb in ((0, 0), (1, 1), (0, 1), (1, 0)):
                for pad in (0, 1):
                    check(oracle, Problem(ta, tb, m, n, k, pad, seed), 1, cfg)
                    seed += 1


def test_every_tile_configuration_gives_the_same_bits(gpu, oracle):
    """The depth order of each element is independent of the kernel's tiling, so every configuration
    returns the oracle's bits."""
    import nnh
    n_cfg = len(nnh.gemm_configs())
    seed = 50000
    for (ta, tb, m, n, k, pad) in ((0, 0, 256, 256, 256, 0), (1, 1, 300, 200, 77, 1), (0, 1, 64, 512, 600, 0),
                                   (1, 0, 512, 64, 2048, 0), (1, 0, 70, 37, 529, 1), (0, 1, 33, 90, 16, 0)):
        p = Problem(ta, tb, m, n, k, pad, seed)
        seed += 1
        for acc in (0, 1):
            want = oracle_sgemm(oracle, p, acc)
            for cfg in range(n_cfg):
                got = gpu_sgemm(p, acc, config=cfg)
                assert bits_equal(got, want), (cfg, p.args(), acc, first_diff(got, want))


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1)])
def test_baseline_config1_512(gpu, oracle, ta, tb):
    """512^3 from seed 0 (A filled first, then B, uniform [-1, 1]); NN, A^T B, A B^T.
    Whole output bit-identical to nn-cpp, and within 4 K 2^-24 sum|a||b| of the fp64 product."""
    n = 512
    a, b = synth.uniform_operands(0, [(n, n), (n, n)])
    p = Problem(ta, tb, n, n, n, 0, 0)
    p.a, p.b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    p.c = np.zeros((n, n), np.float32)
    got = check(oracle, p, 0)
    assert within_fp64_bound(got, p, 0, oracle)


@pytest.mark.parametrize("m,n,k", [(1024, 1024, 1024), (2048, 2048, 2048), (4096, 4096, 4096),
                                   (8192, 8192, 8192), (64, 4096, 4096), (4096, 4096, 64)])
def test_baseline_config5_sampled(gpu, oracle, m, n, k):
    """BASELINE config 5 at full size, seed 4: 512 sampled elements (corners, edges, random) bit-identical
    to nn-cpp's arithmetic, repeated launches bitwise equal."""
    import torch

    import nnh
    a, b = synth.uniform_operands(4, [(m, k), (k, n)])
    da, db = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    dc = torch.empty((m, n), device="cuda")
    nnh.sgemm(0, 0, m, n, k, da, k, db, n, dc, n, 0)
    dc2 = torch.empty_like(dc)
    nnh.sgemm(0, 0, m, n, k, da, k, db, n, dc2, n, 0)
    torch.cuda.synchronize()
    assert torch.equal(dc.view(torch.int32), dc2.view(torch.int32))
    rng = np.random.default_rng(m * 7 + n * 3 + k)
    rows = np.concatenate([[0, 0, m - 1, m - 1, m // 2], rng.integers(0, m, 507)])
    cols = np.concatenate([[0, n - 1, 0, n - 1, n // 2], rng.integers(0, n, 507)])
    got = dc.cpu().numpy()[rows, cols]
    want = oracle.sgemm_at(0, 0, m, n, k, a, k, b, n, 0, rows, cols)
    assert got.tobytes() == want.tobytes(), first_diff(got, want)


@pytest.mark.parametrize("m,n,k", [(1024, 1024, 1024), (2048, 2048, 2048), (4096, 4096, 4096),
                                   (8192, 8192, 8192), (64, 4096, 4096), (4096, 4096, 64)])
def test_baseline_config5_whole_output_vs_nncpp(gpu, ref, m, n, k):
    """BASELINE config 5 at full size, seed 4: every element of nn::matmul's output bit-identical to nn-cpp's own
    compiled nn::matmul (oracle/_ref, its AVX2 build, multithreaded) on the same host buffers."""
    import torch

    import nnh
    a, b = synth.uniform_operands(4, [(m, k), (k, n)])
    rc, want = ref.matmul(a, b, False, False)
    assert rc == 0
    da, db = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    dc = torch.empty((m, n), device="cuda")
    nnh.sgemm(0, 0, m, n, k, da, k, db, n, dc, n, 0)
    got = dc.cpu().numpy()
    assert_same(got, want, f"{m}x{n}x{k}")


def _subnormal_problem(ta, tb, m, n, k, seed):
    """Operands whose products and running sums are subnormal: op(A) and op(B) entries near 2^-80 .. 2^-68
    (products 2^-160 .. 2^-136), except at depth indices 5 and 260, where op(A) holds subnormal values (about
    2^-135 .. 2^-130) and op(B) values in [2^-5, 1], so a subnormal operand makes a subnormal product that dominates
    each output (a flush of subnormal inputs would lose it); signs are mixed and C holds subnormals (accumulate)."""
    p = Problem(ta, tb, m, n, k, 2, seed)
    rng = np.random.default_rng(seed)
    opa = (p.a[:k, :m].T if ta else p.a[:m, :k]).astype(np.float64)
    opb = (p.b[:n, :k].T if tb else p.b[:k, :n]).astype(np.float64)
    opa = np.ldexp(opa, rng.integers(-80, -68, opa.shape))
    opb = np.ldexp(opb, rng.integers(-80, -68, opb.shape))
    for k0 in (5, 260):
        if k0 < k:
            opa[:, k0] = np.ldexp(np.sign(opa[:, k0]) * rng.uniform(1, 2, m), rng.integers(-135, -130, m))
            opb[k0, :] = np.ldexp(np.sign(opb[k0, :]) * rng.uniform(1, 2, n), rng.integers(-5, 0, n))
    opa, opb = opa.astype(np.float32), opb.astype(np.float32)
    if ta:
        p.a[:k, :m] = opa.T
    else:
        p.a[:m, :k] = opa
    if tb:
        p.b[:n, :k] = opb.T
    else:
        p.b[:k, :n] = opb
    p.c[:m, :n] = np.ldexp(p.c[:m, :n].astype(np.float64), rng.integers(-140, -128, (m, n))).astype(np.float32)
    return p


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_subnormal_operands_and_sums(gpu, oracle, ta, tb):
    """nn-cpp's AVX2 chain keeps subnormals (no flush to zero), and so must the MFMA chain: subnormal operands,
    products and running sums, every tile configuration, with and without accumulate, bit for bit."""
    import nnh
    p = _subnormal_problem(ta, tb, 37, 41, 300, 77 + 2 * ta + tb)
    vals = np.concatenate([p.a.ravel(), p.b.ravel()])
    assert np.any((vals != 0) & (np.abs(vals) < np.finfo(np.float32).tiny))
    for acc in (0, 1):
        want = oracle_sgemm(oracle, p, acc)
        out = want[: p.m, : p.n]
        assert np.any((out != 0) & (np.abs(out) < np.finfo(np.float32).tiny)), "no subnormal result: test too weak"
        for cfg in range(len(nnh.gemm_configs())):
            got = gpu_sgemm(p, acc, config=cfg)
            assert bits_equal(got, want), (cfg, acc, first_diff(got, want))


@pytest.mark.parametrize("m,n,k", [(1024, 1024, 1024), (64, 4096, 4096), (4096, 4096, 64)])
def test_baseline_config5_whole_output(gpu, oracle, m, n, k):
    """BASELINE config 5 shapes, seed 4: every element bit-identical to nn-cpp (its compiled sgemm when present,
    else the oracle), not a sample."""
    import torch

    import nnh
    from pyoracle import Reference, reference_available
    a, b = synth.uniform_operands(4, [(m, k), (k, n)])
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    da, db = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    dc = torch.empty((m, n), device="cuda")
    nnh.sgemm(0, 0, m, n, k, da, k, db, n, dc, n, 0)
    torch.cuda.synchronize()
    c0 = np.zeros((m, n), np.float32)
    if reference_available():
        r = Reference()
        r.set_threads(8)
        want = r.sgemm(0, 0, m, n, k, a, k, b, n, c0, n, 0)
    else:
        want = oracle.sgemm(0, 0, m, n, k, a, k, b, n, c0, n, 0)
    got = dc.cpu().numpy()
    assert bits_equal(got, want), first_diff(got, want)


def _batched_cut_case(ta, tb, m, n, k, pad, count, seed):
    """count matrices of A (each its own values), one B shared by all (batch stride 0), C per matrix."""
    a_rows, a_cols = (k, m) if ta else (m, k)
    b_rows, b_cols = (n, k) if tb else (k, n)
    lda, ldb, ldc = a_cols + pad, b_cols + pad, n + pad
    vals = synth.mt19937_uniform(seed, count * a_rows * a_cols + b_rows * b_cols + count * m * n, -1.0, 1.0)
    a = np.full((count, a_rows, lda), SENTINEL, np.float32)
    a[:, :, :a_cols] = vals[: count * a_rows * a_cols].reshape(count, a_rows, a_cols)
    o = count * a_rows * a_cols
    b = np.full((b_rows, ldb), SENTINEL, np.float32)
    b[:, :b_cols] = vals[o: o + b_rows * b_cols].reshape(b_rows, b_cols)
    o += b_rows * b_cols
    c = np.full((count, m, ldc), SENTINEL, np.float32)
    c[:, :, :n] = vals[o:].reshape(count, m, n)
    return a, lda, b, ldb, c, ldc


def _pieces4_config():
    import nnh
    return next(i for i, nm in enumerate(nnh.gemm_configs()) if nm.startswith("mfma pieces 16x16x4"))


@pytest.mark.parametrize("force4", [0, 1])
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_depth_cut_in_one_launch(gpu, oracle, ta, tb, force4):
    """Cut products of at most 16 pieces run as one launch, one wave per piece, that adds the pieces in LDS (no
    partial sums in HBM): a batch of 64 products of 64 x 64 x 1200 (10 pieces, the last one 48 deep) with B shared
    by the batch, 16-byte and element loads, accumulate; 16 pieces (the most one launch takes); and one product of
    40 x 50 x 1000 (8 pieces, ragged tiles) with each bias mode and ReLU with its mask. Every element against the
    oracle, bit for bit; force4 runs them all on the 16x16x4 MFMA pieces kernel (four depth steps of every chain
    per instruction), otherwise the kernel the shape is routed to."""
    import torch

    import nnh
    cfg = _pieces4_config() if force4 else -1
    m, n, k, count = 64, 64, 1200, 64
    assert nnh.workspace_size("sgemm", m, n, k, count) == 0
    for pad in (0, 1):
        a, lda, b, ldb, c, ldc = _batched_cut_case(ta, tb, m, n, k, pad, count, 90000 + 10 * pad + 2 * ta + tb)
        batch = nnh.make_batch((count,), (a[0].size,), (0,), (c[0].size,))
        for acc in (0, 1):
            da, db, dc = (torch.from_numpy(x).cuda() for x in (a, b, np.array(c, copy=True)))
            nnh.sgemm_batched(ta, tb, m, n, k, da, lda, db, ldb, dc, ldc, acc, batch, None, cfg)
            got = dc.cpu().numpy()
            for i in range(count):
                want = oracle.sgemm(ta, tb, m, n, k, np.ascontiguousarray(a[i]), lda, b, ldb,
                                    np.ascontiguousarray(c[i]), ldc, acc)
                assert bits_equal(got[i], want), (pad, acc, i, first_diff(got[i], want))
    p = Problem(ta, tb, 33, 70, 2048, 1, 90500 + 2 * ta + tb)
    assert nnh.workspace_size("sgemm", 33, 70, 2048, 1) == 0
    for acc in (0, 1):
        got, want = gpu_sgemm(p, acc, cfg), oracle_sgemm(oracle, p, acc)
        assert bits_equal(got, want), ("16 pieces", acc, first_diff(got, want))
    m, n, k = 40, 50, 1000
    assert nnh.workspace_size("sgemm", m, n, k, 1) == 0
    p = Problem(ta, tb, m, n, k, 0, 91000 + 2 * ta + tb)
    bias_col = synth.mt19937_uniform(91010, n, -1.0, 1.0)
    bias_row = synth.mt19937_uniform(91011, m, -1.0, 1.0)
    for mode, bias in ((nnh.BIAS_NONE, None), (nnh.BIAS_COL, bias_col), (nnh.BIAS_ROW, bias_row)):
        for relu in (False, True):
            for acc in (0, 1):
                dbias = torch.from_numpy(bias).cuda() if bias is not None else None
                dalive = torch.full((m, p.ldc), 7, dtype=torch.uint8, device="cuda")
                ep = nnh.make_epilogue(mode, dbias, relu, dalive if relu else None)
                got = gpu_sgemm(p, acc, cfg, epilogue=ep)
                want = oracle_sgemm(oracle, p, acc).copy()
                v = want[:m, :n]
                if mode == nnh.BIAS_COL:
                    v += bias_col[None, :]
                elif mode == nnh.BIAS_ROW:
                    v += bias_row[:, None]
                if relu:
                    on = v > 0
                    v[~on] = 0.0
                    alive = dalive.cpu().numpy()
                    assert np.array_equal(alive[:, :n], on.astype(np.uint8)), (mode, acc)
                    assert np.all(alive[:, n:] == 7)
                assert bits_equal(got, want), (mode, relu, acc, first_diff(got, want))


def _valu_pieces_config():
    import nnh
    return next(i for i, nm in enumerate(nnh.gemm_configs()) if nm.startswith("valu pieces"))


@pytest.mark.parametrize("force_valu", [0, 1])
@pytest.mark.parametrize("tb", [0, 1])
def test_four_piece_cuts(gpu, oracle, tb, force_valu):
    """nn-cpp's cut at a depth of 512 (four 128-deep pieces, e.g. config 2's 256 x 256 x 512 layer): on the kernel
    the shape is routed to (the 16x16x4 MFMA pieces kernel with 16-byte loads of its k-contiguous operands when
    aligned, else the VALU pieces kernel), and forced onto the VALU pieces kernel (every piece of an output as a chain
    in one lane). Ragged and tile-aligned m x n, aligned and padded rows (pad), accumulate, a batch sharing B, and each
    bias mode with ReLU and its mask. Every element against the oracle."""
    import torch

    import nnh
    cfg = _valu_pieces_config() if force_valu else -1
    seed = 93000 + 100 * tb
    for m, n, pad in ((256, 256, 0), (37, 90, 1), (128, 16, 0), (50, 41, 1), (16, 4096, 0)):
        for acc in (0, 1):
            p = Problem(0, tb, m, n, 512, pad, seed)
            seed += 1
            got, want = gpu_sgemm(p, acc, cfg), oracle_sgemm(oracle, p, acc)
            assert bits_equal(got, want), ((m, n, pad), acc, first_diff(got, want))
    m, n, k, count = 64, 32, 512, 8
    for pad in (0, 1):
        a, lda, b, ldb, c, ldc = _batched_cut_case(0, tb, m, n, k, pad, count, seed + pad)
        batch = nnh.make_batch((count,), (a[0].size,), (0,), (c[0].size,))
        for acc in (0, 1):
            da, db, dc = (torch.from_numpy(x).cuda() for x in (a, b, np.array(c, copy=True)))
            nnh.sgemm_batched(0, tb, m, n, k, da, lda, db, ldb, dc, ldc, acc, batch, None, cfg)
            got = dc.cpu().numpy()
            for i in range(count):
                want = oracle.sgemm(0, tb, m, n, k, np.ascontiguousarray(a[i]), lda, b, ldb,
                                    np.ascontiguousarray(c[i]), ldc, acc)
                assert bits_equal(got[i], want), (pad, acc, i, first_diff(got[i], want))
    m, n = 40, 60
    p = Problem(0, tb, m, n, 512, 0, seed + 7)
    bias_col = synth.mt19937_uniform(seed + 8, n, -1.0, 1.0)
    bias_row = synth.mt19937_uniform(seed + 9, m, -1.0, 1.0)
    for mode, bias in ((nnh.BIAS_NONE, None), (nnh.BIAS_COL, bias_col), (nnh.BIAS_ROW, bias_row)):
        for relu in (False, True):
            for acc in (0, 1):
                dbias = torch.from_numpy(bias).cuda() if bias is not None else None
                dalive = torch.full((m, p.ldc), 7, dtype=torch.uint8, device="cuda")
                ep = nnh.make_epilogue(mode, dbias, relu, dalive if relu else None)
                got = gpu_sgemm(p, acc, cfg, epilogue=ep)
                want = oracle_sgemm(oracle, p, acc).copy()
                v = want[:m, :n]
                if mode == nnh.BIAS_COL:
                    v += bias_col[None, :]
                elif mode == nnh.BIAS_ROW:
                    v += bias_row[:, None]
                if relu:
                    on = v > 0
                    v[~on] = 0.0
                    alive = dalive.cpu().numpy()
                    assert np.array_equal(alive[:, :n], on.astype(np.uint8)), (mode, acc)
                    assert np.all(alive[:, n:] == 7)
                assert bits_equal(got, want), (mode, relu, acc, first_diff(got, want))

"""nn::batchnorm (training mode, with and without its folded ReLU) and nn::layernorm on the GPU (nnh_batchnorm_*,
nnh_layernorm_*) against the oracle, bit for bit: outputs, statistics, and every gradient, fresh and added to, at
the shapes of nn-cpp's cnn_fer and transformer_tiny workloads and on the edges of the kernels (rows with an
eight-element tail, rows longer than a staging chunk, one element per row, unaligned buffers, many samples)."""
import numpy as np
import pytest

from helpers import assert_same

pytestmark = pytest.mark.gpu

EPS = 1e-5


def dev_off(a, offset, dtype=None):
    """A device copy of a placed `offset` elements into a larger buffer (offset 1 breaks 16-byte alignment)."""
    import torch
    a = np.ascontiguousarray(a)
    t = torch.empty(a.size + offset, dtype=torch.from_numpy(a[:0]).dtype, device="cuda")
    t[offset:] = torch.from_numpy(a.ravel()).cuda()
    return t


def host(t, offset, shape, dtype=np.float32):
    return t[offset:].cpu().numpy().view(dtype).reshape(shape)


def run_bn(x, w, b, relu, g, offset=0, old=None, want=(True, True, True)):
    """Forward, then the backward rule (fresh, or added to `old` = (dx, dw, db)) through the C ABI."""
    import torch

    import nnh
    L = nnh.lib()
    N, Cc = x.shape[:2]
    S = x.size // max(1, N * Cc) if N * Cc else int(np.prod(x.shape[2:]))
    xd, wd, bd, gd = dev_off(x, offset), dev_off(w, 0), dev_off(b, 0), dev_off(g, offset)
    y = dev_off(np.full(x.shape, np.nan, np.float32), offset)
    alive = dev_off(np.full(x.shape, 7, np.uint8), offset) if relu else None
    mean, var, inv = (dev_off(np.full(Cc, np.nan, np.float32), 0) for _ in range(3))
    nnh.check(L.nnh_batchnorm_forward(nnh._ptr(xd, offset), N, Cc, S, nnh._ptr(wd), nnh._ptr(bd), EPS, int(relu),
                                      nnh._ptr(y, offset), nnh._ptr(alive, offset) if relu else None, nnh._ptr(mean),
                                      nnh._ptr(var), nnh._ptr(inv), nnh._stream(None)))
    first = old is None
    bufs = []
    for i, (shape, off) in enumerate(((x.shape, offset), ((Cc,), 0), ((Cc,), 0))):
        if not want[i]:
            bufs.append(None)
            continue
        init = np.full(shape, np.nan, np.float32) if first else old[i]
        bufs.append(dev_off(init, off))
    nnh.check(L.nnh_batchnorm_backward(nnh._ptr(gd, offset), nnh._ptr(xd, offset),
                                       nnh._ptr(alive, offset) if relu else None, nnh._ptr(wd), nnh._ptr(mean),
                                       nnh._ptr(inv), N, Cc, S,
                                       nnh._ptr(bufs[0], offset) if want[0] else None, int(first),
                                       nnh._ptr(bufs[1]) if want[1] else None, int(first),
                                       nnh._ptr(bufs[2]) if want[2] else None, int(first), nnh._stream(None)))
    torch.cuda.synchronize()
    out = dict(y=host(y, offset, x.shape), mean=host(mean, 0, (Cc,)), var=host(var, 0, (Cc,)),
               inv=host(inv, 0, (Cc,)))
    out["alive"] = host(alive, offset, x.shape, np.uint8) if relu else None
    for name, t, shape, off in (("dx", bufs[0], x.shape, offset), ("dw", bufs[1], (Cc,), 0),
                                ("db", bufs[2], (Cc,), 0)):
        out[name] = host(t, off, shape) if t is not None else None
    return out


def bn_inputs(shape, seed):
    rng = np.random.default_rng(seed)
    Cc = shape[1]
    x = rng.uniform(-3, 5, shape).astype(np.float32)
    w = rng.uniform(0.5, 1.5, Cc).astype(np.float32)
    b = rng.uniform(-1, 1, Cc).astype(np.float32)
    g = rng.normal(size=shape).astype(np.float32)
    return x, w, b, g


BN_CASES = [
    ((64, 16, 48, 48), 1),   # cnn_fer: Conv-BN-ReLU stacks at batch 64
    ((64, 32, 24, 24), 1),
    ((64, 64, 12, 12), 1),
    ((32, 8, 28, 28), 0),
    ((4, 3, 5, 5), 0),       # S = 25: an eight-element tail, element-wise loads
    ((3, 2, 2049), 1),       # rows longer than a staging chunk, with a tail
    ((5, 2, 8), 0),
    ((1, 3, 1, 1), 0),       # one element per channel
    ((300, 7), 1),           # BatchNorm1d: many samples, S = 1
    ((2, 5, 1024), 1),       # exactly one staging chunk (forward) and more than one (backward)
]


@pytest.mark.parametrize("shape,relu", BN_CASES)
def test_batchnorm_matches_oracle(oracle, shape, relu):
    x, w, b, g = bn_inputs(shape, sum(shape) + relu)
    y, alive, mean, var, inv = oracle.batchnorm_forward(x, w, b, EPS, relu)
    got = run_bn(x, w, b, relu, g)
    tag = f"batchnorm {shape} relu={relu}"
    assert_same(got["y"], y, tag + " y")
    assert_same(got["mean"], mean, tag + " mean")
    assert_same(got["var"], var, tag + " var")
    assert_same(got["inv"], inv, tag + " inv_std")
    if relu:
        assert np.array_equal(got["alive"], alive), tag + " alive"
    dx, dw, db = oracle.batchnorm_backward(g, x, alive, w, mean, inv)
    assert_same(got["dx"], dx, tag + " dx")
    assert_same(got["dw"], dw, tag + " dw")
    assert_same(got["db"], db, tag + " db")
    # the same rule adding into existing gradients
    rng = np.random.default_rng(7)
    old = (rng.normal(size=shape).astype(np.float32), rng.normal(size=shape[1]).astype(np.float32),
           rng.normal(size=shape[1]).astype(np.float32))
    got2 = run_bn(x, w, b, relu, g, old=old)
    dx2, dw2, db2 = oracle.batchnorm_backward(g, x, alive, w, mean, inv, old[0], False, old[1], False, old[2], False)
    assert_same(got2["dx"], dx2, tag + " dx added")
    assert_same(got2["dw"], dw2, tag + " dw added")
    assert_same(got2["db"], db2, tag + " db added")


@pytest.mark.parametrize("shape,relu", [((8, 3, 12, 12), 1), ((4, 3, 5, 5), 0), ((2, 2, 37), 1)])
def test_batchnorm_unaligned_buffers_and_gradient_subsets(oracle, shape, relu):
    """x, y, g and dx one float off 16-byte alignment (the element-wise paths), and the backward with only some
    gradients wanted."""
    x, w, b, g = bn_inputs(shape, 11 + relu)
    y, alive, mean, var, inv = oracle.batchnorm_forward(x, w, b, EPS, relu)
    dx, dw, db = oracle.batchnorm_backward(g, x, alive, w, mean, inv)
    got = run_bn(x, w, b, relu, g, offset=1)
    assert_same(got["y"], y, "unaligned y")
    assert_same(got["dx"], dx, "unaligned dx")
    for want in ((False, True, True), (True, False, False), (False, False, True)):
        got = run_bn(x, w, b, relu, g, want=want)
        for name, ref_val, wanted in (("dx", dx, want[0]), ("dw", dw, want[1]), ("db", db, want[2])):
            if wanted:
                assert_same(got[name], ref_val, f"{name} with want={want}")
            else:
                assert got[name] is None


def test_batchnorm_special_values(oracle):
    """NaN and infinities in one channel make that channel's statistics NaN (as in the reference) and leave the
    other channels exact; zero-variance channels go through 1 / sqrt(eps)."""
    x, w, b, g = bn_inputs((4, 4, 3, 3), 21)
    x[1, 0, 1, 1] = np.nan
    x[2, 1, 0, 0] = np.inf
    x[:, 2] = 1.5
    for relu in (0, 1):
        y, alive, mean, var, inv = oracle.batchnorm_forward(x, w, b, EPS, relu)
        got = run_bn(x, w, b, relu, g)
        assert_same(got["y"], y, "special y", nan_equal=True)
        assert_same(got["mean"], mean, "special mean", nan_equal=True)
        dx, dw, db = oracle.batchnorm_backward(g, x, alive, w, mean, inv)
        assert_same(got["dx"], dx, "special dx", nan_equal=True)
        assert_same(got["dw"], dw, "special dw", nan_equal=True)
        assert_same(got["db"], db, "special db", nan_equal=True)


def test_batchnorm_bitwise_repeat():
    x, w, b, g = bn_inputs((64, 16, 48, 48), 31)
    a, c = run_bn(x, w, b, 1, g), run_bn(x, w, b, 1, g)
    for k in ("y", "mean", "var", "dx", "dw", "db"):
        assert a[k].tobytes() == c[k].tobytes(), k


def run_ln(x, gm, bt, g, offset=0, old=None, want=(True, True, True)):
    import torch

    import nnh
    L = nnh.lib()
    D = x.shape[-1]
    R = x.size // D
    xd, gmd, btd, gd = dev_off(x, offset), dev_off(gm, 0), dev_off(bt, 0), dev_off(g, offset)
    y = dev_off(np.full(x.shape, np.nan, np.float32), offset)
    mean, inv = dev_off(np.full(R, np.nan, np.float32), 0), dev_off(np.full(R, np.nan, np.float32), 0)
    nnh.check(L.nnh_layernorm_forward(nnh._ptr(xd, offset), R, D, nnh._ptr(gmd), nnh._ptr(btd), EPS,
                                      nnh._ptr(y, offset), nnh._ptr(mean), nnh._ptr(inv), nnh._stream(None)))
    first = old is None
    bufs = []
    for i, (shape, off) in enumerate(((x.shape, offset), ((D,), 0), ((D,), 0))):
        if not want[i]:
            bufs.append(None)
            continue
        bufs.append(dev_off(np.full(shape, np.nan, np.float32) if first else old[i], off))
    nnh.check(L.nnh_layernorm_backward(nnh._ptr(gd, offset), nnh._ptr(xd, offset), nnh._ptr(gmd), nnh._ptr(mean),
                                       nnh._ptr(inv), R, D, nnh._ptr(bufs[0], offset) if want[0] else None, int(first),
                                       nnh._ptr(bufs[1]) if want[1] else None, int(first),
                                       nnh._ptr(bufs[2]) if want[2] else None, int(first), nnh._stream(None)))
    torch.cuda.synchronize()
    out = dict(y=host(y, offset, x.shape), mean=host(mean, 0, (R,)), inv=host(inv, 0, (R,)))
    for name, t, shape, off in (("dx", bufs[0], x.shape, offset), ("dgamma", bufs[1], (D,), 0),
                                ("dbeta", bufs[2], (D,), 0)):
        out[name] = host(t, off, shape) if t is not None else None
    return out


def ln_inputs(shape, seed):
    rng = np.random.default_rng(seed)
    D = shape[-1]
    return (rng.uniform(-2, 3, shape).astype(np.float32), rng.uniform(0.5, 1.5, D).astype(np.float32),
            rng.uniform(-1, 1, D).astype(np.float32), rng.normal(size=shape).astype(np.float32))


LN_CASES = [(16, 64, 64), (40, 30, 16), (3, 7, 33), (2, 515), (1, 4), (300, 1), (256, 512), (1023, 17), (1025, 8),
            (3001, 40), (8, 1024, 512), (1201, 7),
            # wide rows: from D = 5460 the backward's LDS block holds no row (ln_backward_kernel, a thread per row and
            # per column); from D = 16384 the forward's neither (ln_forward_kernel)
            (3, 5459), (3, 5460), (2, 8192), (2, 16383), (2, 16384), (3, 20000), (5, 16385)]


@pytest.mark.parametrize("shape", LN_CASES)
def test_layernorm_matches_oracle(oracle, shape):
    """transformer_tiny's {16, 64, 64} first; rows of odd length (element-wise loads), one column, many rows."""
    x, gm, bt, g = ln_inputs(shape, sum(shape))
    y, mean, inv = oracle.layernorm_forward(x, gm, bt, EPS)
    got = run_ln(x, gm, bt, g)
    tag = f"layernorm {shape}"
    assert_same(got["y"], y, tag + " y")
    assert_same(got["mean"], mean, tag + " mean")
    assert_same(got["inv"], inv, tag + " inv_std")
    dx, dg, db = oracle.layernorm_backward(g, x, gm, mean, inv)
    assert_same(got["dx"], dx, tag + " dx")
    assert_same(got["dgamma"], dg, tag + " dgamma")
    assert_same(got["dbeta"], db, tag + " dbeta")
    rng = np.random.default_rng(3)
    D = shape[-1]
    old = (rng.normal(size=shape).astype(np.float32), rng.normal(size=D).astype(np.float32),
           rng.normal(size=D).astype(np.float32))
    got2 = run_ln(x, gm, bt, g, old=old)
    dx2, dg2, db2 = oracle.layernorm_backward(g, x, gm, mean, inv, old[0], False, old[1], False, old[2], False)
    assert_same(got2["dx"], dx2, tag + " dx added")
    assert_same(got2["dgamma"], dg2, tag + " dgamma added")
    assert_same(got2["dbeta"], db2, tag + " dbeta added")


def test_layernorm_unaligned_and_subsets(oracle):
    x, gm, bt, g = ln_inputs((16, 64, 64), 41)
    y, mean, inv = oracle.layernorm_forward(x, gm, bt, EPS)
    dx, dg, db = oracle.layernorm_backward(g, x, gm, mean, inv)
    got = run_ln(x, gm, bt, g, offset=1)
    assert_same(got["y"], y, "unaligned y")
    assert_same(got["dx"], dx, "unaligned dx")
    for want in ((False, True, False), (True, False, False), (False, False, True)):
        got = run_ln(x, gm, bt, g, want=want)
        for name, ref_val, wanted in (("dx", dx, want[0]), ("dgamma", dg, want[1]), ("dbeta", db, want[2])):
            if wanted:
                assert_same(got[name], ref_val, f"{name} with want={want}")


@pytest.mark.parametrize("shape", [(3, 5461), (2, 16384)])
def test_layernorm_wide_rows_unaligned(oracle, shape):
    """The wide-row kernels on buffers one float past 16-byte alignment."""
    x, gm, bt, g = ln_inputs(shape, 77)
    y, mean, inv = oracle.layernorm_forward(x, gm, bt, EPS)
    dx, dg, db = oracle.layernorm_backward(g, x, gm, mean, inv)
    got = run_ln(x, gm, bt, g, offset=1)
    assert_same(got["y"], y, f"{shape} unaligned y")
    assert_same(got["dx"], dx, f"{shape} unaligned dx")
    assert_same(got["dgamma"], dg, f"{shape} dgamma")
    assert_same(got["dbeta"], db, f"{shape} dbeta")


def test_norm_shape_errors():
    import nnh
    L = nnh.lib()
    # layernorm over an empty last axis: the reference divides by zero; refused before anything is enqueued
    assert L.nnh_layernorm_forward(None, 4, 0, None, None, EPS, None, None, None, nnh._stream(None)) == nnh.ERR_INVALID
    # no channels: nothing to do
    assert L.nnh_batchnorm_forward(None, 4, 0, 3, None, None, EPS, 0, None, None, None, None, None,
                                   nnh._stream(None)) == 0

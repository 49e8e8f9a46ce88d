"""The transformer's element-wise ops on the GPU (nnh_add_forward, nnh_gelu_*, nnh_embedding_*) against the
oracle, bit for bit: GELU over a sweep that crosses the tanh clamp and every special value, fresh and added
gradients; add with a broadcast row, on aligned and unaligned buffers and in place; embedding rows gathered and the
gradient table built in token order with repeated ids, fresh and added to, over more tokens than one staging pass."""
import ctypes as C

import numpy as np
import pytest

from helpers import assert_same

pytestmark = pytest.mark.gpu


def dev(a, offset=0):
    """A device copy of a placed `offset` elements into a larger buffer (offset 1 breaks 16-byte alignment)."""
    import torch
    a = np.ascontiguousarray(a)
    t = torch.empty(a.size + offset, dtype=torch.from_numpy(a[:0]).dtype, device="cuda")
    t[offset:] = torch.from_numpy(a.ravel()).cuda()
    return t


def host(t, offset, shape):
    return t[offset:].cpu().numpy().reshape(shape)


def gelu_inputs(n, seed):
    rng = np.random.default_rng(seed)
    x = np.concatenate([rng.normal(size=n).astype(np.float32) * 3,
                        np.linspace(-12, 12, 4001).astype(np.float32),
                        np.array([0, -0.0, 1e-30, -1e-30, 1e4, -1e4, np.inf, -np.inf, np.nan], np.float32)])
    return x, rng.normal(size=x.size).astype(np.float32)


@pytest.mark.parametrize("n,offset", [(0, 0), (1, 0), (64 * 256, 0), (64 * 256, 1), (300000, 0)])
def test_gelu_bitwise(gpu, oracle, n, offset):
    import torch

    import nnh
    L = nnh.lib()
    x, g = gelu_inputs(n, n)
    want_y, want_th = oracle.gelu_forward(x)
    xd, gd = dev(x, offset), dev(g, offset)
    y, th = dev(np.full(x.size, np.nan, np.float32), offset), dev(np.full(x.size, np.nan, np.float32), offset)
    nnh.check(L.nnh_gelu_forward(nnh._ptr(xd, offset), x.size, nnh._ptr(y, offset), nnh._ptr(th, offset),
                                 nnh._stream(None)))
    dx = dev(np.full(x.size, np.nan, np.float32), offset)
    nnh.check(L.nnh_gelu_backward(nnh._ptr(xd, offset), nnh._ptr(th, offset), nnh._ptr(gd, offset), x.size,
                                  nnh._ptr(dx, offset), 1, nnh._stream(None)))
    torch.cuda.synchronize()
    assert_same(host(y, offset, x.shape), want_y, "gelu y", nan_equal=True)
    assert_same(host(th, offset, x.shape), want_th, "gelu tanh", nan_equal=True)
    want_dx = oracle.gelu_backward(x, want_th, g)
    assert_same(host(dx, offset, x.shape), want_dx, "gelu dx", nan_equal=True)
    # added to an existing gradient (the second use of the same activation)
    nnh.check(L.nnh_gelu_backward(nnh._ptr(xd, offset), nnh._ptr(th, offset), nnh._ptr(gd, offset), x.size,
                                  nnh._ptr(dx, offset), 0, nnh._stream(None)))
    torch.cuda.synchronize()
    assert_same(host(dx, offset, x.shape), oracle.gelu_backward(x, want_th, g, want_dx, False), "gelu dx added",
                nan_equal=True)


def test_gelu_backward_in_place_over_g(gpu, oracle):
    """dx may be g itself (each element reads its g before writing dx)."""
    import torch

    import nnh
    L = nnh.lib()
    x, g = gelu_inputs(5000, 3)
    _, th = oracle.gelu_forward(x)
    xd, thd, gd = dev(x), dev(th), dev(g)
    nnh.check(L.nnh_gelu_backward(nnh._ptr(xd), nnh._ptr(thd), nnh._ptr(gd), x.size, nnh._ptr(gd), 1,
                                  nnh._stream(None)))
    torch.cuda.synchronize()
    assert_same(gd.cpu().numpy(), oracle.gelu_backward(x, th, g), "gelu dx over g", nan_equal=True)


@pytest.mark.parametrize("outer,inner,offset", [(1, 1, 0), (7, 3, 0), (512, 64, 0), (512, 64, 1), (64, 256, 0),
                                                (3, 100003, 0), (1000, 4, 0)])
def test_add_broadcast_bitwise(gpu, outer, inner, offset):
    """y = a + b with b one row broadcast over the leading axes (nn::add's suffix broadcast): one rounding per
    element, so numpy's float32 sum is the reference's."""
    import torch

    import nnh
    L = nnh.lib()
    rng = np.random.default_rng(outer * 7 + inner)
    a = rng.normal(size=(outer, inner)).astype(np.float32)
    b = rng.normal(size=inner).astype(np.float32)
    ad, bd = dev(a, offset), dev(b, offset)
    y = dev(np.full(a.shape, np.nan, np.float32), offset)
    nnh.check(L.nnh_add_forward(nnh._ptr(ad, offset), nnh._ptr(bd, offset), outer, inner, nnh._ptr(y, offset),
                                nnh._stream(None)))
    torch.cuda.synchronize()
    assert_same(host(y, offset, a.shape), a + b, "add")
    # in place: y = a
    nnh.check(L.nnh_add_forward(nnh._ptr(ad, offset), nnh._ptr(bd, offset), outer, inner, nnh._ptr(ad, offset),
                                nnh._stream(None)))
    torch.cuda.synchronize()
    assert_same(host(ad, offset, a.shape), a + b, "add in place")


def test_add_rejects_overlaps(gpu):
    import torch

    import nnh
    L = nnh.lib()
    t = torch.zeros(64, device="cuda")
    with pytest.raises(nnh.NnhError):
        nnh.check(L.nnh_add_forward(nnh._ptr(t), nnh._ptr(t, 32), 2, 16, nnh._ptr(t, 40), nnh._stream(None)))
    with pytest.raises(nnh.NnhError):  # y shifted by one element against a
        nnh.check(L.nnh_add_forward(nnh._ptr(t), nnh._ptr(t, 48), 2, 16, nnh._ptr(t, 1), nnh._stream(None)))


@pytest.mark.parametrize("V,D,count,offset", [(64, 64, 512, 0), (64, 64, 4096, 0), (5, 3, 2500, 1), (1, 8, 10, 0),
                                              (1000, 1, 3000, 0), (64, 64, 0, 0), (7, 130, 2000, 0), (3, 64, 1500, 1),
                                              (2, 200, 1025, 0)])
def test_embedding_bitwise(gpu, oracle, V, D, count, offset):
    import torch

    import nnh
    L = nnh.lib()
    rng = np.random.default_rng(V * 31 + count)
    w = rng.normal(size=(V, D)).astype(np.float32)
    rows = rng.integers(0, V, count).astype(np.int32)
    g = rng.normal(size=(count, D)).astype(np.float32)
    wd, rd, gd = dev(w, offset), dev(rows, offset), dev(g, offset)
    y = dev(np.full((count, D), np.nan, np.float32), offset)
    nnh.check(L.nnh_embedding_forward(nnh._ptr(wd, offset), V, D, nnh._ptr(rd, offset), count, nnh._ptr(y, offset),
                                      nnh._stream(None)))
    dw = dev(np.full((V, D), np.nan, np.float32), offset)
    nnh.check(L.nnh_embedding_backward(nnh._ptr(gd, offset), nnh._ptr(rd, offset), count, V, D, nnh._ptr(dw, offset),
                                       1, nnh._stream(None)))
    torch.cuda.synchronize()
    assert_same(host(y, offset, (count, D)), w[rows], "embedding y")
    # with an addend broadcast over the rows (a transformer's positions): the lookup, then the float add
    T = max([t for t in range(1, 65) if count % t == 0] or [1])
    pe = rng.normal(size=(T, D)).astype(np.float32)
    ped = dev(pe, offset)
    y2 = dev(np.full((count, D), np.nan, np.float32), offset)
    nnh.check(L.nnh_embedding_add_forward(nnh._ptr(wd, offset), V, D, nnh._ptr(rd, offset), count, nnh._ptr(ped, offset),
                                          T, nnh._ptr(y2, offset), nnh._stream(None)))
    torch.cuda.synchronize()
    if count:
        assert_same(host(y2, offset, (count, D)), w[rows] + np.tile(pe, (count // T, 1)), "embedding + addend")
    want = oracle.embedding_backward(g, rows, V, D)
    assert_same(host(dw, offset, (V, D)), want, "embedding dw")
    nnh.check(L.nnh_embedding_backward(nnh._ptr(gd, offset), nnh._ptr(rd, offset), count, V, D, nnh._ptr(dw, offset),
                                       0, nnh._stream(None)))
    torch.cuda.synchronize()
    assert_same(host(dw, offset, (V, D)), oracle.embedding_backward(g, rows, V, D, want, False), "embedding dw added")


def test_embedding_errors(gpu):
    import torch

    import nnh
    L = nnh.lib()
    t = torch.zeros(64, device="cuda")
    r = torch.zeros(4, dtype=torch.int32, device="cuda")
    with pytest.raises(nnh.ShapeError):  # an empty table has no row for any id
        nnh.check(L.nnh_embedding_forward(nnh._ptr(t), 0, 4, nnh._ptr(r), 4, nnh._ptr(t), nnh._stream(None)))
    with pytest.raises(nnh.NnhError):  # y over the table
        nnh.check(L.nnh_embedding_forward(nnh._ptr(t), 4, 4, nnh._ptr(r), 2, nnh._ptr(t, 8), nnh._stream(None)))
    p = torch.zeros(64, device="cuda")
    with pytest.raises(nnh.ShapeError):  # the addend's rows must divide the ids' count
        nnh.check(L.nnh_embedding_add_forward(nnh._ptr(t), 4, 4, nnh._ptr(r), 4, nnh._ptr(p), 3, nnh._ptr(t, 32),
                                              nnh._stream(None)))
    with pytest.raises(nnh.NnhError):  # y over the addend
        nnh.check(L.nnh_embedding_add_forward(nnh._ptr(t), 4, 4, nnh._ptr(r), 4, nnh._ptr(p), 2, nnh._ptr(p, 4),
                                              nnh._stream(None)))


def test_embedding_backward_keeps_negative_zero(gpu, oracle):
    """Added to an existing gradient of -0 with gradients of -0, every entry stays -0: tokens of other rows add
    nothing (not even +0)."""
    import torch

    import nnh
    L = nnh.lib()
    V, D, count = 6, 70, 700
    rows = np.random.default_rng(3).integers(0, V - 1, count).astype(np.int32)  # the last row gets no token
    g = np.full((count, D), -0.0, np.float32)
    old = np.full((V, D), -0.0, np.float32)
    gd, rd, dw = dev(g), dev(rows), dev(old)
    nnh.check(L.nnh_embedding_backward(nnh._ptr(gd), nnh._ptr(rd), count, V, D, nnh._ptr(dw), 0, nnh._stream(None)))
    torch.cuda.synchronize()
    want = oracle.embedding_backward(g, rows, V, D, old, False)
    assert np.all(np.signbit(want))
    assert_same(dw.cpu().numpy().reshape(V, D), want, "embedding dw of -0")


def test_zero_many(gpu):
    """nnh_zero_many (an optimizer's zero_grad over its parameters in one launch per 64 buffers): 70 buffers of
    sizes 0 to 70,001 carved from one allocation with gaps (two launches; empty buffers first, last and between),
    every buffer +0 afterwards (no -0) and every gap untouched; overlapping buffers are refused."""
    import torch

    import nnh
    rng = np.random.default_rng(5)
    sizes = [0, 1, 3, 64, 70001] + list(rng.integers(1, 5000, 35)) + [0, 0] + list(rng.integers(1, 900, 27)) + [0]
    total = sum(sizes) + 7 * len(sizes)
    base = torch.full((total,), -0.0, device="cuda")
    views, gaps, off = [], [], 0
    for n in sizes:
        views.append(base[off:off + n])
        off += n
        gaps.append((off, off + 7))
        off += 7
    base[:] = torch.from_numpy(rng.normal(size=total).astype(np.float32)).cuda()
    before = base.cpu().numpy().copy()
    nnh.zero_many(views)
    torch.cuda.synchronize()
    after = base.cpu().numpy()
    off = 0
    for n in sizes:
        seg = after[off:off + n]
        assert np.all(seg == 0) and not np.any(np.signbit(seg)), n
        off += n
        assert np.array_equal(after[off:off + 7].view(np.uint32), before[off:off + 7].view(np.uint32))
        off += 7
    with pytest.raises(nnh.NnhError):
        nnh.zero_many([base[0:10], base[5:20]])


@pytest.mark.parametrize("n,first0,first1", [(1, 1, 1), (1000, 1, 0), (70001, 0, 1), (4096, 0, 0)])
def test_add_to_grad2_matches_two_calls(gpu, n, first0, first1):
    """nnh_add_to_grad2 (an add node's backward into both operands in one launch) gives each gradient the bits of its
    own nnh_add_to_grad call: a fresh one stores src + 0 (-0 becomes +0), an existing one adds src. Signed zeros,
    infinities and NaN in src and in the old gradients."""
    import torch

    import nnh
    L = nnh.lib()
    rng = np.random.default_rng(n)
    src = rng.standard_normal(n).astype(np.float32)
    old0 = rng.standard_normal(n).astype(np.float32)
    old1 = rng.standard_normal(n).astype(np.float32)
    if n > 8:
        src[:4] = [-0.0, 0.0, np.inf, np.nan]
        old0[4:6] = [-0.0, -np.inf]
        old1[1:3] = [-0.0, np.inf]
    ds = dev(src)
    got = [dev(old0), dev(old1)]
    want = [dev(old0), dev(old1)]
    ptr = lambda t: C.c_void_p(t.data_ptr())
    assert L.nnh_add_to_grad2(ptr(got[0]), first0, ptr(got[1]), first1, ptr(ds), n, None) == 0
    assert L.nnh_add_to_grad(ptr(want[0]), ptr(ds), n, first0, None) == 0
    assert L.nnh_add_to_grad(ptr(want[1]), ptr(ds), n, first1, None) == 0
    torch.cuda.synchronize()
    for i in range(2):
        assert_same(got[i].cpu().numpy(), want[i].cpu().numpy(), ("gradient", i), nan_equal=True)
    with np.errstate(all="ignore"):
        ref0 = src + np.float32(0) if first0 else old0 + src
    assert_same(got[0].cpu().numpy(), ref0, "gradient 0 vs numpy", nan_equal=True)

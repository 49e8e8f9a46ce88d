"""The packed flag forms (nnh_conv2d_relu_forward_packed, nnh_conv2d_relu_maxpool2d_forward_packed,
nnh_conv2d_backward_packed, nnh_maxpool2d_backward_packed): a network's first layer keeps its ReLU flags one bit per
output and its 2 x 2 pool's maxima as 2-bit window positions. The values and gradients are bit for bit those of the
byte forms and of the oracle's conv2d_relu / maxpool2d (the reference's ops.cpp conv2d_relu and maxpool2d); the bits
are np.packbits of the oracle's alive bytes (little bit order) and the positions decode to the oracle's plane
offsets. Covered: config 3's conv1, ragged sample counts, row widths whose quads split unevenly over a wave (W = 12,
28, 40), the widest row (W = 256), kh != kw, 8 input channels of a 1 x 1 kernel, NaN / -inf / -0 inputs and a
channel of all-zero outputs (ties keep the window's first position)."""
import numpy as np
import pytest

from helpers import assert_same
from nnh import synth

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits_of(alive):
    return np.packbits(np.ascontiguousarray(alive).reshape(-1), bitorder="little")


def unpack_argmax2(a2, planes, h, w):
    """Plane offsets of the 2-bit positions: window (ph, pw) of plane p at bits 2 (pw % 4) of byte
    (p (h / 2) + ph) ceil(w / 8) + pw / 4; position r * 2 + c is row 2 ph + r, column 2 pw + c."""
    ph, pw, rb = h // 2, w // 2, (w + 7) // 8
    j = np.arange(pw)
    slot = (a2.reshape(planes, ph, rb)[:, :, j // 4] >> (2 * (j % 4)).astype(np.uint8)) & 3
    return ((2 * np.arange(ph)[None, :, None] + slot // 2) * w + 2 * j[None, None, :] + slot % 2).astype(np.uint32)


def operands(case, seed):
    N, Cin, H, W, Cout, kh, kw, pad = case
    x = synth.mt19937_uniform(seed, N * Cin * H * W, -1.0, 1.0).reshape(N, Cin, H, W)
    x[0, 0, 0, :3] = [np.nan, -np.inf, -0.0]
    w = synth.normal(seed + 1, (Cout, Cin, kh, kw))
    b = synth.mt19937_uniform(seed + 2, Cout, -0.5, 0.5)
    b[0] = -8.0  # a channel whose outputs are all zero after the ReLU (ties in every window)
    return x, w, b


# (N, Cin, H, W, Cout, kh, kw, pad)
CONV_CASES = [
    (128, 1, 28, 28, 32, 3, 3, 1),   # config 3's conv1
    (3, 1, 28, 28, 32, 3, 3, 1),     # a ragged sample count
    (3, 1, 12, 8, 5, 3, 3, 1),       # 96 outputs per plane
    (2, 1, 10, 16, 7, 1, 3, 1),      # kh != kw: 12 x 16 outputs
    (2, 8, 8, 8, 24, 1, 1, 0),       # K = 8 from 8 input channels of a 1 x 1 kernel
    (2, 2, 6, 4, 12, 1, 3, 1),       # one quad per row, Cin 2
]


@pytest.mark.parametrize("case", CONV_CASES)
def test_conv_relu_packed_matches_byte_form(gpu, oracle, case):
    import torch

    import nnh
    x, w, b = operands(case, 11 + case[3])
    N, Cin, H, W, Cout, kh, kw, pad = case
    assert nnh.conv2d_packed_supported(x.shape, w.shape, 1, pad), case
    dx_, dw_, db_ = dev(x), dev(w), dev(b)
    y, bits = nnh.conv2d_relu_forward_packed(dx_, dw_, db_, 1, pad)
    yb, alive = nnh.conv2d_forward(dx_, dw_, db_, 1, pad, True)
    wy, wa = oracle.conv2d_forward(x, w, b, 1, pad, True)
    assert_same(host(y), wy, ("y", case))
    assert np.array_equal(host(bits), bits_of(wa)), case
    assert np.array_equal(host(bits), bits_of(host(alive))), case
    # the backward from the bits: every subset of gradients, fresh and accumulated, against the byte form
    gr = synth.normal(case[4] + 5, tuple(y.shape))
    old = synth.normal(case[4] + 6, x.shape)
    for want in ((1, 1, 1), (1, 0, 0), (0, 1, 0), (0, 0, 1), (0, 1, 1)):
        for first in (True, False):
            outs = []
            for packed in (True, False):
                dx = (torch.full(x.shape, float("nan"), device="cuda") if first else dev(old)) if want[0] else None
                dw = (torch.full(w.shape, float("nan"), device="cuda") if first else dev(w * 0.5)) if want[1] else None
                db = (torch.full(b.shape, float("nan"), device="cuda") if first else dev(b * 0.5)) if want[2] else None
                if packed:
                    nnh.conv2d_backward_packed(dev(gr), dx_, dw_, bits, 1, pad, dx, first, dw, first, db, first)
                else:
                    nnh.conv2d_backward(dev(gr), dx_, dw_, alive, 1, pad, dx, first, dw, first, db, first)
                outs.append([None if t is None else host(t) for t in (dx, dw, db)])
            wdx, wdw, wdb = oracle.conv2d_backward(gr, x, w, wa, 1, pad, dx=None if first else old, dx_first=first)
            wanted = (wdx, wdw if first else w * np.float32(0.5) + wdw, wdb if first else b * np.float32(0.5) + wdb)
            for i, name in enumerate(("dx", "dw", "db")):
                if want[i]:
                    assert_same(outs[0][i], outs[1][i], (name, "vs bytes", case, want, first))
                    if i == 0 or first:
                        # NaN from the NaN / -inf inputs: any NaN matches (its payload depends on the order of the
                        # products that meet it); every other value bit for bit
                        assert_same(outs[0][i], wanted[i], (name, "vs oracle", case, want, first), nan_equal=True)


# (N, H, W, Cout): Cin 1, 3 x 3, padding 1, then the 2 x 2 stride-2 pool
POOL_CASES = [
    (128, 28, 28, 32),   # config 3's conv1 + pool1: 7 quads per row, 63 lanes of a wave
    (3, 28, 28, 9),
    (2, 10, 12, 7),      # 3 quads per row
    (2, 8, 4, 4),        # one quad per row
    (2, 16, 32, 9),      # 8 quads per row: whole waves
    (3, 6, 40, 3),       # 10 quads per row: 60 lanes of a wave
    (1, 4, 256, 2),      # the widest row
]


@pytest.mark.parametrize("case", POOL_CASES)
def test_conv_relu_pool_packed_matches_byte_form(gpu, oracle, case):
    import torch

    import nnh
    N, H, W, Cout = case
    x, w, b = operands((N, 1, H, W, Cout, 3, 3, 1), 40 + W)
    assert nnh.conv2d_packed_supported(x.shape, w.shape, 1, 1, with_pool=True), case
    dx_, dw_, db_ = dev(x), dev(w), dev(b)
    y, bits, pooled, a2 = nnh.conv2d_relu_maxpool2d_forward_packed(dx_, dw_, db_, 1, 1)
    yb, alive, pb, arg = nnh.conv2d_relu_maxpool2d_forward(dx_, dw_, db_, 1, 1, 2, 2)
    wy, wa = oracle.conv2d_forward(x, w, b, 1, 1, True)
    wp, warg = oracle.maxpool2d_forward(wy, 2, 2)
    assert_same(host(y), wy, ("y", case))
    assert_same(host(pooled), wp, ("pooled", case))
    assert np.array_equal(host(bits), bits_of(wa)), case
    assert np.array_equal(host(bits), bits_of(host(alive))), case
    offs = unpack_argmax2(host(a2), N * Cout, H, W)
    assert np.array_equal(offs.reshape(-1), warg.reshape(-1)), case
    assert np.array_equal(offs.reshape(-1), host(arg).view(np.uint32).reshape(-1)), case
    # the pool's backward from the positions, fresh and accumulated, against the 32-bit offsets' and the oracle
    g = synth.normal(70 + W, tuple(pooled.shape))
    old = synth.normal(71 + W, tuple(y.shape))
    L, P, st = nnh.lib(), nnh._ptr, nnh._stream(None)
    for first in (True, False):
        d1 = torch.full(y.shape, float("nan"), device="cuda") if first else dev(old)
        d2 = torch.full(y.shape, float("nan"), device="cuda") if first else dev(old)
        gd = dev(g)
        nnh.maxpool2d_backward_packed(gd, a2, d1, first)
        nnh.check(L.nnh_maxpool2d_backward(P(gd), P(arg), N, Cout, H, W, 2, 2, P(d2), int(first), st))
        got = host(d1)
        assert_same(got, host(d2), ("pool dx vs offsets", case, first))
        want = oracle.maxpool2d_backward(g, warg, wy.shape, 2, 2, dx=None if first else old, first=first)
        assert_same(got, want, ("pool dx vs oracle", case, first))
    # and the conv's backward from the bits
    gr = synth.normal(72 + W, tuple(y.shape))
    outs = []
    for packed in (True, False):
        dx, dw, db = (torch.full(t.shape, float("nan"), device="cuda") for t in (x, w, b))
        if packed:
            nnh.conv2d_backward_packed(dev(gr), dx_, dw_, bits, 1, 1, dx, True, dw, True, db, True)
        else:
            nnh.conv2d_backward(dev(gr), dx_, dw_, alive, 1, 1, dx, True, dw, True, db, True)
        outs.append([host(t) for t in (dx, dw, db)])
    for i, name in enumerate(("dx", "dw", "db")):
        assert_same(outs[0][i], outs[1][i], (name, case))


def test_packed_refusals(gpu):
    """Geometries and pointers the packed forms do not take are refused before anything is launched; the queries
    agree with the calls."""
    import torch

    import nnh
    L, P, st = nnh.lib(), nnh._ptr, nnh._stream(None)
    x = torch.zeros(2 * 28 * 28 + 4, device="cuda")
    w = torch.zeros(32 * 9, device="cuda")
    b = torch.zeros(32, device="cuda")
    y = torch.zeros(2 * 32 * 784 + 4, device="cuda")
    bits = torch.zeros(2 * 32 * 784 // 8 + 16, dtype=torch.uint8, device="cuda")
    p = torch.zeros(2 * 32 * 196 + 4, device="cuda")
    a2 = torch.zeros(2 * 32 * 14 * 4 + 16, dtype=torch.uint8, device="cuda")
    f = L.nnh_conv2d_relu_forward_packed
    fp = L.nnh_conv2d_relu_maxpool2d_forward_packed
    assert f(P(x), 2, 1, 28, 28, P(w), 32, 3, 3, P(b), 1, 1, P(y), P(bits), st) == nnh.OK
    assert f(P(x), 2, 1, 28, 28, P(w), 32, 3, 3, P(b), 1, 1, P(y, 1), P(bits), st) == nnh.ERR_INVALID  # y unaligned
    assert f(P(x, 2), 2, 1, 28, 28, P(w), 32, 3, 3, P(b), 1, 1, P(y), P(bits), st) == nnh.ERR_INVALID  # x unaligned
    assert f(P(x), 2, 1, 28, 28, P(w), 32, 3, 3, P(b), 2, 1, P(y), P(bits), st) == nnh.ERR_INVALID     # stride 2
    assert f(P(x), 2, 1, 28, 28, P(w), 32, 3, 3, P(b), 1, 1, P(y), None, st) == nnh.ERR_INVALID
    assert f(P(x), 2, 1, 28, 28, P(w), 32, 3, 3, P(b), 1, 1, P(y), P(y), st) == nnh.ERR_ALIAS
    assert fp(P(x), 2, 1, 28, 28, P(w), 32, 3, 3, P(b), 1, 1, P(y), P(bits), P(p), P(a2), st) == nnh.OK
    assert fp(P(x), 2, 1, 28, 28, P(w), 32, 3, 3, P(b), 1, 1, P(y), P(bits), P(p, 1), P(a2), st) == nnh.ERR_INVALID
    assert fp(P(x), 2, 1, 28, 28, P(w), 32, 3, 3, P(b), 1, 1, P(y), P(bits), P(p), P(bits), st) == nnh.ERR_ALIAS
    assert fp(P(x), 2, 1, 27, 28, P(w), 32, 3, 3, P(b), 1, 1, P(y), P(bits), P(p), P(a2), st) == nnh.ERR_INVALID
    g = torch.zeros(2 * 33 * 784 + 4, device="cuda")  # room for the Cout 33 call's extent (refused, not read)
    dx = torch.zeros(2 * 784, device="cuda")
    bw = L.nnh_conv2d_backward_packed
    assert bw(P(g), P(x), P(w), P(bits), 2, 1, 28, 28, 32, 3, 3, 1, 1, P(dx), 1, None, 1, None, 1, st) == nnh.OK
    assert bw(P(g, 1), P(x), P(w), P(bits), 2, 1, 28, 28, 32, 3, 3, 1, 1, P(dx), 1, None, 1, None, 1, st) == \
        nnh.ERR_INVALID  # g unaligned
    assert bw(P(g), P(x), P(w), None, 2, 1, 28, 28, 32, 3, 3, 1, 1, P(dx), 1, None, 1, None, 1, st) == nnh.ERR_INVALID
    assert bw(P(g), P(x), P(w), P(bits), 2, 1, 28, 28, 33, 3, 3, 1, 1, P(dx), 1, None, 1, None, 1, st) == \
        nnh.ERR_INVALID  # Cout 33
    torch.cuda.synchronize()

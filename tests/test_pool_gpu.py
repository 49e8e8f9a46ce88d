"""nn::maxpool2d on the GPU (nnh_maxpool2d_forward / _backward) against the oracle, bit for bit: outputs, argmax
offsets and input gradients (fresh and accumulated), at config 3's size (2 x 2, stride 2 on conv1's output) and on
the special cases the reference defines (ties, NaN, windows of -inf, overlapping windows)."""
import numpy as np
import pytest

from helpers import assert_same
from nnh import synth

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run_pool(x, k, s, g, old=None, offset=0):
    """Forward and backward through the C ABI; offset shifts the buffers by that many floats (alignment)."""
    import torch

    import nnh
    L = nnh.lib()
    N, C, H, W = x.shape
    ho, wo = (H - k) // s + 1, (W - k) // s + 1
    xb = torch.empty(x.size + offset, device="cuda")
    xb[offset:] = dev(x).ravel()
    y = torch.empty(N * C * ho * wo + offset, device="cuda")
    arg = torch.empty(N * C * ho * wo + offset, dtype=torch.int32, device="cuda")
    nnh.check(L.nnh_maxpool2d_forward(nnh._ptr(xb, offset), N, C, H, W, k, s, nnh._ptr(y, offset),
                                      C_ptr(arg, offset), nnh._stream(None)))
    dx = dev(old if old is not None else np.full(x.shape, np.nan, np.float32))
    nnh.check(L.nnh_maxpool2d_backward(nnh._ptr(dev(g)), C_ptr(arg, offset), N, C, H, W, k, s, nnh._ptr(dx),
                                       int(old is None), nnh._stream(None)))
    torch.cuda.synchronize()
    return (y[offset:].cpu().numpy().reshape(N, C, ho, wo), arg[offset:].cpu().numpy().view(np.uint32)
            .reshape(N, C, ho, wo), dx.cpu().numpy())


def C_ptr(t, offset=0):
    import ctypes
    return ctypes.c_void_p(t.data_ptr() + 4 * offset)


CASES = [
    (128, 32, 28, 28, 2, 2, 81, 0),   # config 3: conv1's output pooled for conv2
    (2, 3, 9, 7, 3, 2, 82, 1),
    (1, 2, 6, 6, 3, 1, 83, 1),
    (3, 2, 5, 5, 2, 1, 84, 1),
    (2, 2, 7, 9, 2, 2, 85, 1),
    (2, 4, 8, 12, 2, 2, 86, 1),       # the two-output kernel with -inf and NaN windows
    (1, 1, 1, 1, 1, 1, 87, 0),
    (1, 2, 40, 36, 2, 2, 88, 1),      # 360 windows a plane: a kept-0 window past a wave's first pass
]


def inputs(case):
    N, C, H, W, k, s, seed, specials = case
    ho, wo = (H - k) // s + 1, (W - k) // s + 1
    x, g = synth.uniform_operands(seed, [(N, C, H, W), (N, C, ho, wo)])
    x = np.array(x, copy=True)
    if specials:
        x = (np.round(x * 4) / 4).astype(np.float32)
        x[0, 0, H - k:H, W - k:W] = -np.inf
        x[-1, -1, 0:k, 0:k] = np.nan
        x[0, -1, H // 2, W // 2] = np.nan
    return x, np.ascontiguousarray(g), k, s


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("offset", [0, 1])
def test_maxpool_matches_oracle(gpu, oracle, case, offset):
    x, g, k, s = inputs(case)
    y, arg, dx = run_pool(x, k, s, g, offset=offset)
    wy, warg = oracle.maxpool2d_forward(x, k, s)
    assert_same(y, wy, ("y", case, offset))
    assert np.array_equal(arg, warg), ("argmax", case, offset)
    assert_same(dx, oracle.maxpool2d_backward(g, warg, x.shape, k, s), ("dx fresh", case, offset))
    old = synth.normal(case[6] + 1, x.shape)
    _, _, dx2 = run_pool(x, k, s, g, old=old, offset=offset)
    assert_same(dx2, oracle.maxpool2d_backward(g, warg, x.shape, k, s, dx=old, first=False), ("dx acc", case, offset))


def test_maxpool_shape_errors(gpu):
    import nnh
    L = nnh.lib()
    assert L.nnh_maxpool2d_forward(None, 1, 1, 3, 3, 4, 1, None, None, None) == nnh.ERR_SHAPE
    assert L.nnh_maxpool2d_forward(None, 1, 1, 3, 3, 0, 1, None, None, None) == nnh.ERR_SHAPE
    assert L.nnh_maxpool2d_forward(None, 1, 1, 3, 3, 2, 0, None, None, None) == nnh.ERR_SHAPE


FUSED_CASES = [  # (N, Cin, H, W, Cout, k, pad, stride, pool k, pool s, seed, alive, argmax)
    (128, 1, 28, 28, 32, 3, 1, 1, 2, 2, 91, True, True),    # config 3's conv1 -> ReLU -> pool: one kernel
    (3, 2, 12, 8, 5, 3, 1, 1, 2, 2, 92, True, True),        # two input channels, a partial channel group
    (2, 1, 10, 12, 7, 5, 2, 1, 2, 2, 93, False, True),      # 5 x 5, padding 2, no alive flags
    (2, 1, 8, 4, 4, 3, 1, 1, 2, 2, 94, True, False),        # one quad per row (both halos are padding), no argmax
    (2, 1, 9, 8, 4, 3, 1, 1, 2, 2, 95, True, True),         # H odd: the two ops in turn
    (2, 3, 8, 8, 4, 3, 1, 1, 2, 2, 96, True, True),         # Cin (kh + 1) > 8: the two ops in turn
    (2, 1, 8, 8, 4, 3, 1, 1, 3, 2, 97, True, True),         # a 3 x 3 pool: the two ops in turn
]


@pytest.mark.parametrize("case", FUSED_CASES)
def test_conv_relu_maxpool_in_one_pass(oracle, case):
    """nnh_conv2d_relu_maxpool2d_forward gives conv2d_relu's y and alive flags and maxpool2d's output and argmax on
    them, bit for bit, the same as the two ops (nnh_conv2d_forward, nnh_maxpool2d_forward) and as the oracle's
    conv2d_relu and maxpool2d; inputs include -0, NaN and -inf (the ReLU maps them to 0, windows of zeros keep their
    first offset)."""
    import torch

    import nnh
    N, Cin, H, W, Cout, k, pad, stride, pk, ps, seed, want_alive, want_argmax = case
    x, wt, b = synth.uniform_operands(seed, [(N, Cin, H, W), (Cout, Cin, k, k), (Cout,)])
    x = np.array(x, copy=True)
    x[0, 0, 0, :3] = [np.nan, -np.inf, -0.0]
    b = np.array(b, copy=True)
    b[0] = -4.0  # a channel whose outputs are mostly zero after the ReLU: windows of equal zeros
    dx_, dw_, db_ = dev(x), dev(wt), dev(b)
    y, al, p, arg = nnh.conv2d_relu_maxpool2d_forward(dx_, dw_, db_, stride, pad, pk, ps, want_alive, want_argmax)
    y2, al2 = nnh.conv2d_forward(dx_, dw_, db_, stride, pad, True)
    p2, arg2 = nnh.maxpool2d_forward(y2, pk, ps)
    torch.cuda.synchronize()
    wy, wal = oracle.conv2d_forward(x, wt, b, stride, pad, True)
    wp, warg = oracle.maxpool2d_forward(wy, pk, ps)
    assert_same(y.cpu().numpy(), wy, ("y", case))
    assert_same(y.cpu().numpy(), y2.cpu().numpy(), ("y vs two ops", case))
    if want_alive:
        assert np.array_equal(al.cpu().numpy(), wal), case
    assert_same(p.cpu().numpy(), wp, ("pooled", case))
    assert_same(p.cpu().numpy(), p2.cpu().numpy(), ("pooled vs two ops", case))
    if want_argmax:
        assert np.array_equal(arg.cpu().numpy().view(np.uint32), warg), case
        assert np.array_equal(arg.cpu().numpy(), arg2.cpu().numpy()), case

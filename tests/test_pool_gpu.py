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

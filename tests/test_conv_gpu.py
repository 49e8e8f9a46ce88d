"""Parity of nn::conv2d / nn::conv2d_relu (forward and backward), im2col and col2im on the GPU.

Bitwise against nn-cpp's golden outputs and against the oracle at BASELINE config 3 (batch 128: conv1 1->32 on
28x28, conv2 32->64 on 14x14 after 2x2 max-pooling), on both forward paths (direct for a short depth, im2col +
MFMA GEMM for a long one).
"""
import numpy as np
import pytest

from helpers import assert_same
from nnh import synth

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def same(got, want, what):
    assert_same(got, want, what)


def test_conv_golden(gpu):
    import golden_cases as gc
    import torch

    import nnh
    g = np.load(gc.__file__.replace("golden_cases.py", "reference_vectors.npz"))
    for name, spec in gc.CONV_CASES:
        x, w, bias, gr, stride, pad, relu = gc.conv_inputs(spec)
        y, alive = nnh.conv2d_forward(dev(x), dev(w), dev(bias), stride, pad, relu)
        same(host(y), g[f"conv/{name}/y"], name)
        # nn-cpp's leaves add into zero-filled gradients
        dx, dw, db = (torch.zeros(t.shape, device="cuda") for t in (x, w, bias))
        nnh.conv2d_backward(dev(gr), dev(x), dev(w), alive, stride, pad, dx, False, dw, False, db, False)
        for key, t in (("dx", dx), ("dw", dw), ("db", db)):
            same(host(t), g[f"conv/{name}/{key}"], (name, key))


def maxpool2(y):
    N, C, H, W = y.shape
    return y.reshape(N, C, H // 2, 2, W // 2, 2).max(axis=(3, 5))


def config3():
    """x ~ U[0,1] (seed 2); conv weights ~ N(0, sqrt(2 / fan_in)) (Kaiming-normal), zero biases."""
    x = synth.mt19937_uniform(2, 128 * 28 * 28, 0.0, 1.0).reshape(128, 1, 28, 28)
    w1 = (synth.normal(21, (32, 1, 3, 3)) * np.float32(np.sqrt(2.0 / 9))).astype(np.float32)
    w2 = (synth.normal(22, (64, 32, 3, 3)) * np.float32(np.sqrt(2.0 / 288))).astype(np.float32)
    return x, w1, w2


@pytest.mark.parametrize("layer", [1, 2])
def test_baseline_config3(gpu, oracle, layer):
    import torch

    import nnh
    x, w1, w2 = config3()
    b1, b2 = np.zeros(32, np.float32), np.zeros(64, np.float32)
    y1, a1 = oracle.conv2d_forward(x, w1, b1, 1, 1, 1)
    if layer == 1:
        xin, w, b, want_y, want_a = x, w1, b1, y1, a1
    else:
        xin = np.ascontiguousarray(maxpool2(y1))
        w, b = w2, b2
        want_y, want_a = oracle.conv2d_forward(xin, w, b, 1, 1, 1)
    y, alive = nnh.conv2d_forward(dev(xin), dev(w), dev(b), 1, 1, True)
    same(host(y), want_y, f"conv{layer} forward")
    same(host(alive), want_a, f"conv{layer} alive")
    gr = synth.normal(30 + layer, want_y.shape)
    dx, dw, db = (torch.full(t.shape, float("nan"), device="cuda") for t in (xin, w, b))
    nnh.conv2d_backward(dev(gr), dev(xin), dev(w), alive, 1, 1, dx, True, dw, True, db, True)
    wdx, wdw, wdb = oracle.conv2d_backward(gr, xin, w, want_a, 1, 1, dx_first=True)
    same(host(dx), wdx, f"conv{layer} dx")
    same(host(dw), wdw, f"conv{layer} dw")
    same(host(db), wdb, f"conv{layer} db")


def test_direct_and_gemm_paths_match_the_oracle(gpu, oracle):
    """K = Cin*kh*kw <= 32 takes the direct kernel, longer depths one GEMM whose B tiles are gathered from x
    (implicit im2col); both are the reference's chain. Backward (mask, db, dW with gathered columns, dcol and
    col2im) on every case; the last case's forward product takes nn-cpp's depth cut (m n <= 2^16, K = 576)."""
    import torch

    import nnh
    for (N, Cin, H, W, Cout, kk, s, p) in ((3, 3, 11, 9, 40, 3, 1, 1), (3, 4, 11, 9, 40, 3, 1, 1),
                                            (2, 1, 8, 8, 5, 5, 2, 2), (2, 8, 8, 8, 70, 5, 2, 2), (5, 2, 7, 6, 3, 2, 3, 0),
                                            (2, 64, 8, 8, 64, 3, 1, 1)):
        x = synth.mt19937_uniform(N * 100 + Cin, N * Cin * H * W).reshape(N, Cin, H, W)
        w = synth.mt19937_uniform(Cout + 7, Cout * Cin * kk * kk).reshape(Cout, Cin, kk, kk)
        b = synth.mt19937_uniform(Cout + 8, Cout)
        for relu in (False, True):
            y, alive = nnh.conv2d_forward(dev(x), dev(w), dev(b), s, p, relu)
            wy, wa = oracle.conv2d_forward(x, w, b, s, p, relu)
            same(host(y), wy, (N, Cin, Cout, kk, s, p, relu))
            if relu:
                same(host(alive), wa, "alive")
        gr = synth.mt19937_uniform(Cout + 9, wy.size).reshape(wy.shape)
        dx, dw, db = torch.empty(x.shape, device="cuda"), torch.empty(w.shape, device="cuda"), torch.empty(Cout, device="cuda")
        nnh.conv2d_backward(dev(gr), dev(x), dev(w), alive, s, p, dx, True, dw, True, db, True)
        wdx, wdw, wdb = oracle.conv2d_backward(gr, x, w, wa, s, p, dx_first=True)
        for got, want, key in ((dx, wdx, "dx"), (dw, wdw, "dw"), (db, wdb, "db")):
            same(host(got), want, (key, N, Cin, Cout, kk, s, p))


# dx with dcol kept on chip (Ho*Wo <= 256): input-channel groups that do not divide Cin, Cout over several 64-wide
# chunks with a ragged end, strides, rectangular and large kernels, output planes that do not fill a wave; first-layer
# planes (Ho*Wo <= 1024, kh*kw <= 16) in bands of dx rows or whole; and larger planes, which take the batched GEMM and
# col2im. (N, Cin, H, W, Cout, kh, kw, stride, pad)
DX_CASES = [
    (2, 13, 14, 14, 64, 3, 3, 1, 1),    # config 3 conv2's plane; 13 channels: groups of 8 and 5
    (3, 9, 9, 7, 150, 3, 3, 1, 1),      # Cout 150: chunks of 64, 64 and 22
    (2, 5, 11, 11, 7, 5, 5, 2, 2),      # stride 2, 25 taps: 3 channels per group
    (2, 4, 6, 10, 33, 2, 3, 1, 0),      # rectangular kernel, no padding
    (1, 3, 16, 16, 20, 9, 9, 1, 4),     # 81 taps: one channel per group does not fit 80 rows
    (2, 6, 17, 17, 24, 3, 3, 1, 1),     # 289 outputs: bands of 9 and 8 dx rows, one channel per group
    (2, 1, 28, 28, 32, 3, 3, 1, 1),     # config 3's conv1 plane (784 outputs): four bands of seven rows
    (2, 3, 24, 20, 10, 3, 3, 1, 0),     # no padding, 396 outputs: two bands, the first row's taps from row 0 only
    (2, 2, 40, 40, 5, 3, 3, 2, 1),      # stride 2, 400 outputs: sixteen waves, the general tap gather
    (1, 1, 30, 30, 9, 4, 4, 1, 1),      # 16 taps, 841 outputs: six bands of five rows, the general tap gather
    (1, 2, 34, 34, 6, 3, 3, 1, 1),      # 1156 outputs: the GEMM + col2im path
    (2, 8, 8, 8, 512, 3, 3, 1, 1),      # dcol = W^T g (72 x 64 x 512) takes the depth cut: the GEMM + col2im path
]


@pytest.mark.parametrize("case", DX_CASES)
def test_conv_backward_dx_paths(gpu, oracle, case):
    """dx, fresh and accumulated onto an existing gradient, bitwise against the oracle (dW and db too)."""
    import torch

    import nnh
    N, Cin, H, W, Cout, kh, kw, s, p = case
    x = synth.mt19937_uniform(N * 31 + Cin, N * Cin * H * W).reshape(N, Cin, H, W)
    w = synth.normal(Cout + 17, (Cout, Cin, kh, kw))
    b = synth.mt19937_uniform(Cout + 18, Cout)
    y, alive = nnh.conv2d_forward(dev(x), dev(w), dev(b), s, p, True)
    _, wa = oracle.conv2d_forward(x, w, b, s, p, True)
    gr = synth.normal(Cout + 19, tuple(y.shape))
    old = synth.normal(Cout + 20, x.shape)
    for first in (True, False):
        dx = dev(old) if not first else torch.full(x.shape, float("nan"), device="cuda")
        dw, db = torch.empty(w.shape, device="cuda"), torch.empty(Cout, device="cuda")
        nnh.conv2d_backward(dev(gr), dev(x), dev(w), alive, s, p, dx, first, dw, True, db, True)
        wdx, wdw, wdb = oracle.conv2d_backward(gr, x, w, wa, s, p, dx=None if first else old, dx_first=first)
        same(host(dx), wdx, ("dx", case, first))
        same(host(dw), wdw, ("dw", case))
        same(host(db), wdb, ("db", case))


def test_im2col_col2im(gpu, oracle):
    import torch

    import nnh
    for (N, Cin, H, W, kk, s, p) in ((2, 3, 7, 6, 3, 2, 1), (1, 2, 5, 5, 4, 3, 3), (3, 1, 28, 28, 3, 1, 1)):
        x = synth.mt19937_uniform(N + H, N * Cin * H * W).reshape(N, Cin, H, W)
        col = nnh.im2col(dev(x), kk, kk, s, p)
        same(host(col), oracle.im2col(x, kk, kk, s, p), ("im2col", N, Cin, H, W, kk, s, p))
        y = synth.mt19937_uniform(N + W + 1, col.numel()).reshape(tuple(col.shape))
        base = synth.mt19937_uniform(N + W + 2, x.size).reshape(x.shape)
        for first in (True, False):
            d = dev(base)
            nnh.col2im_add(dev(y), d, kk, kk, s, p, first)
            want = oracle.col2im_add(y, np.zeros_like(x) if first else base, kk, kk, s, p)
            same(host(d), want, ("col2im", first))


def test_conv_shape_errors(gpu):
    """ops.cpp:1350-1365: stride > 0, padding >= 0, kernel within the padded input."""
    import torch

    import nnh
    x = torch.zeros((1, 1, 3, 3), device="cuda")
    w = torch.zeros((1, 1, 5, 5), device="cuda")
    b = torch.zeros(1, device="cuda")
    with pytest.raises(nnh.ShapeError):
        nnh.conv2d_forward(x, w, b, 1, 0, False)
    with pytest.raises(nnh.ShapeError):
        nnh.conv2d_forward(x, torch.zeros((1, 1, 2, 2), device="cuda"), b, 0, 0, False)


def test_conv3x3_lds_path(gpu, oracle):
    """3x3, stride 1, padding 1 on planes up to 14 x 14 with Cout a multiple of 32 and H*W a multiple of 4 runs
    as MFMA chains over the input held in LDS: tiny and rectangular planes, one to fifty input channels, several
    32-channel groups, ReLU on and off, special values in x, w and the bias. A product that takes nn-cpp's depth
    cut (Cin = 60: K = 540, 32 x 64 outputs), H*W = 49 and an unaligned y take the GEMM path instead: same bits."""
    import torch

    import nnh
    cases = [(2, 32, 14, 14, 64), (3, 1, 2, 2, 32), (2, 7, 12, 10, 96), (1, 50, 14, 14, 32), (2, 3, 9, 4, 32),
             (1, 60, 8, 8, 32), (2, 3, 7, 7, 32)]
    for ci, (N, Cin, H, W, Cout) in enumerate(cases):
        x = synth.mt19937_uniform(300 + ci, N * Cin * H * W).reshape(N, Cin, H, W) * 2 - 1
        w = synth.normal(310 + ci, (Cout, Cin, 3, 3))
        b = synth.mt19937_uniform(320 + ci, Cout) - np.float32(0.5)
        for relu in (False, True):
            y, alive = nnh.conv2d_forward(dev(x), dev(w), dev(b), 1, 1, relu)
            wy, wa = oracle.conv2d_forward(x, w, b, 1, 1, relu)
            same(host(y), wy, (N, Cin, H, W, Cout, relu))
            if relu:
                same(host(alive), wa, ("alive", N, Cin, H, W, Cout))
    # special values: an infinite or NaN weight or input, -0 inputs and biases; a padding tap is fma(w, 0, acc)
    N, Cin, H, W, Cout = 2, 5, 14, 14, 64
    x = synth.mt19937_uniform(330, N * Cin * H * W).reshape(N, Cin, H, W)
    x[0, 1, 5, 5], x[1, 2, 0, 0], x[1, 3, 13, 13], x[0, 4, 7, 2] = np.inf, np.nan, -0.0, -np.inf
    w = synth.normal(331, (Cout, Cin, 3, 3))
    w[3, 0, 0, 0], w[17, 2, 1, 1], w[40, 4, 2, 2], w[63, 1, 0, 2] = np.inf, np.nan, -0.0, -np.inf
    b = synth.mt19937_uniform(332, Cout)
    b[5], b[6] = -0.0, 0.0
    for relu in (False, True):
        y, alive = nnh.conv2d_forward(dev(x), dev(w), dev(b), 1, 1, relu)
        wy, wa = oracle.conv2d_forward(x, w, b, 1, 1, relu)
        same(host(y), wy, ("special values", relu))
        if relu:
            same(host(alive), wa, "special values alive")
    # an output view that is not 16-byte aligned: the GEMM path
    N, Cin, H, W, Cout = 2, 4, 14, 14, 32
    x = synth.mt19937_uniform(340, N * Cin * H * W).reshape(N, Cin, H, W)
    w = synth.normal(341, (Cout, Cin, 3, 3))
    b = synth.mt19937_uniform(342, Cout)
    buf = torch.zeros(N * Cout * H * W + 1, device="cuda")
    yv = buf[1:]
    dx, dw, db = dev(x), dev(w), dev(b)  # held until the kernel has run
    rc = nnh.lib().nnh_conv2d_forward(nnh._ptr(dx), N, Cin, H, W, nnh._ptr(dw), Cout, 3, 3, nnh._ptr(db), 1, 1,
                                      0, nnh._ptr(yv), None, nnh._stream(None))
    nnh.check(rc)
    wy, _ = oracle.conv2d_forward(x, w, b, 1, 1, False)
    same(host(yv).reshape(wy.shape), wy, "unaligned y")


def test_conv3x3_weight_gradient_lds_path(gpu, oracle):
    """The per-sample weight gradients of 3x3, stride 1, padding 1 convolutions on planes up to 14 x 14 with Cout
    a multiple of 64 run as MFMA chains over the gradient rows and the padded input held in LDS, then the ordered
    sum over samples: several 64-channel groups, one to 42 input channels (a ragged last group of 16 k), tiny and
    rectangular planes, with and without the ReLU mask, accumulating gradients, special values. The same kernel
    masks the gradient (the masked gradient then feeds dx) and takes the per-sample bias sums, so dx and db are
    checked too, also with only some of the three gradients asked for. Cout a multiple of 16 but not of 64 (16 as in
    cnn_mnist's conv2, 32, 80) runs a last group with zero rows past Cout. Planes whose size is not a multiple of 4
    and a gradient that is not 16-byte aligned take the gathered GEMM instead."""
    import torch

    import nnh
    cases = [(3, 32, 14, 14, 64, True), (2, 1, 2, 2, 64, False), (2, 7, 12, 11, 128, True), (1, 42, 14, 14, 64, True),
             (3, 5, 9, 4, 64, False), (2, 3, 14, 14, 32, True), (2, 3, 7, 7, 64, True), (2, 4, 6, 6, 64, False),
             (3, 8, 14, 14, 16, True), (2, 5, 14, 14, 80, True), (2, 2, 4, 4, 48, False)]
    for ci, (N, Cin, H, W, Cout, relu) in enumerate(cases):
        x = synth.mt19937_uniform(400 + ci, N * Cin * H * W).reshape(N, Cin, H, W) * 2 - 1
        w = synth.normal(410 + ci, (Cout, Cin, 3, 3))
        b = synth.mt19937_uniform(420 + ci, Cout) - np.float32(0.5)
        if ci == 2:
            x[0, 1, 3, 3], x[1, 6, 11, 10], x[1, 0, 0, 0] = np.inf, -0.0, np.nan
        y, alive = nnh.conv2d_forward(dev(x), dev(w), dev(b), 1, 1, relu)
        wy, wa = oracle.conv2d_forward(x, w, b, 1, 1, relu)
        same(host(y), wy, ("forward", ci))
        gr = synth.normal(430 + ci, wy.shape)
        for first in (True, False):
            dx0 = synth.mt19937_uniform(440 + ci, x.size).reshape(x.shape)
            dw0 = synth.mt19937_uniform(450 + ci, w.size).reshape(w.shape)
            db0 = synth.mt19937_uniform(460 + ci, Cout)
            dx, dw, db = dev(dx0), dev(dw0), dev(db0)
            gd = dev(gr)
            if ci == 7:  # the gradient one float past a 16-byte boundary
                gd = torch.empty(gr.size + 1, dtype=torch.float32, device="cuda")[1:].view(gr.shape).copy_(gd)
            nnh.conv2d_backward(gd, dev(x), dev(w), alive if relu else None, 1, 1, dx, first, dw, first, db, first)
            wdx, wdw, wdb = oracle.conv2d_backward(gr, x, w, wa if relu else None, 1, 1, dx=None if first else dx0,
                                                   dx_first=first)
            if not first:
                wdw, wdb = dw0 + wdw, db0 + wdb
            else:
                wdw, wdb = wdw + np.float32(0), wdb + np.float32(0)
            for got, want, key in ((dx, wdx, "dx"), (dw, wdw, "dw"), (db, wdb, "db")):
                assert_same(host(got), want.astype(np.float32), (ci, N, Cin, H, W, Cout, relu, first, key),
                            nan_equal=(ci == 2))
        # a subset of the gradients: dW alone, dW and db without dx, dx and db without dW
        wdx, wdw, wdb = oracle.conv2d_backward(gr, x, w, wa if relu else None, 1, 1)
        for want_dx, want_dw, want_db in ((False, True, False), (False, True, True), (True, False, True)):
            dx = dev(np.zeros(x.shape, np.float32)) if want_dx else None
            dw = dev(np.zeros(w.shape, np.float32)) if want_dw else None
            db = dev(np.zeros(Cout, np.float32)) if want_db else None
            nnh.conv2d_backward(dev(gr), dev(x), dev(w), alive if relu else None, 1, 1, dx, True, dw, True, db, True)
            for got, want, key in ((dx, wdx, "dx"), (dw, wdw + np.float32(0), "dw"), (db, wdb + np.float32(0), "db")):
                if got is not None:
                    assert_same(host(got), want.astype(np.float32),
                                (ci, N, Cin, H, W, Cout, relu, want_dx, want_dw, want_db, key), nan_equal=(ci == 2))


def test_same_width_quad_path(gpu, oracle):
    """Stride 1, kw = 2 pad + 1, W % 4 == 0 takes the 4-pixels-per-lane direct kernel: every pad 0..4, several
    input channels, Cout not a multiple of the channel group, kh != kw, rows that straddle waves (W = 28: a wave
    of 64 lanes ends mid-row), and an unaligned y (the scalar kernel then)."""
    import torch

    import nnh
    # (the direct kernels take depths Cin*kh*kw <= 32; pads 3 and 4 reach them with one-row kernels)
    cases = ((4, 1, 28, 28, 32, 3, 3, 1), (3, 2, 9, 12, 7, 1, 1, 0), (2, 1, 10, 8, 19, 5, 5, 2),
             (2, 1, 13, 20, 9, 1, 7, 3), (1, 2, 12, 16, 5, 1, 9, 4), (3, 2, 11, 24, 6, 5, 3, 1),
             (2, 3, 6, 4, 12, 1, 3, 1))
    for (N, Cin, H, W, Cout, kh, kw, p) in cases:
        x = synth.mt19937_uniform(N * 31 + W, N * Cin * H * W).reshape(N, Cin, H, W)
        w = synth.mt19937_uniform(Cout * 3 + kh, Cout * Cin * kh * kw).reshape(Cout, Cin, kh, kw)
        b = synth.mt19937_uniform(Cout + 9, Cout)
        for relu in (False, True):
            y, alive = nnh.conv2d_forward(dev(x), dev(w), dev(b), 1, p, relu)
            wy, wa = oracle.conv2d_forward(x, w, b, 1, p, relu)
            same(host(y), wy, (N, Cin, H, W, Cout, kh, kw, p, relu))
            if relu:
                same(host(alive), wa, ("alive", N, Cin, H, W, Cout, kh, kw, p))
    # Inf, NaN and -0 weights: a padding tap is fma(w, 0, acc), so an infinite weight makes the border NaN
    N, Cin, H, W, Cout = 2, 1, 8, 8, 4
    x = synth.mt19937_uniform(5, N * H * W).reshape(N, Cin, H, W)
    x[0, 0, 3, 3] = -0.0
    w = synth.mt19937_uniform(6, Cout * 9).reshape(Cout, Cin, 3, 3)
    w[0, 0, 0, 0], w[1, 0, 2, 2], w[2, 0, 1, 1], w[3, 0, 1, 0] = np.inf, np.nan, -0.0, -np.inf
    b = np.array([0.0, -0.0, 1.0, -1.0], np.float32)
    for relu in (False, True):
        y, alive = nnh.conv2d_forward(dev(x), dev(w), dev(b), 1, 1, relu)
        wy, wa = oracle.conv2d_forward(x, w, b, 1, 1, relu)
        same(host(y), wy, ("special values", relu))
    # an output view that is not 16-byte aligned falls back to the scalar kernel with the same bits
    x = synth.mt19937_uniform(8, 2 * 1 * 12 * 12).reshape(2, 1, 12, 12)
    w = synth.mt19937_uniform(9, 5 * 9).reshape(5, 1, 3, 3)
    b = synth.mt19937_uniform(10, 5)
    buf = torch.zeros(2 * 5 * 144 + 1, device="cuda")
    yv = buf[1:]
    dx, dw, db = dev(x), dev(w), dev(b)  # held until the kernel has run
    rc = nnh.lib().nnh_conv2d_forward(nnh._ptr(dx), 2, 1, 12, 12, nnh._ptr(dw), 5, 3, 3, nnh._ptr(db), 1, 1,
                                      1, nnh._ptr(yv), None, nnh._stream(None))
    nnh.check(rc)
    wy, _ = oracle.conv2d_forward(x, w, b, 1, 1, True)
    same(host(yv).reshape(wy.shape), wy, "unaligned y")


# First layers: K = Cin*kh*kw <= 16 with Cout <= 32, stride 1, Ho*Wo a multiple of 4 and a padded input plane of up
# to 2048 floats take one kernel per sample for db, dW and dx (conv_first); other short-depth layers take the
# per-sample db and dW kernel (conv_dwp) and a dx kernel that masks g itself. (N, Cin, H, W, Cout, kh, kw, stride,
# pad)
DWP_CASES = [
    (4, 1, 28, 28, 32, 3, 3, 1, 1),     # config 3's conv1
    (3, 1, 13, 13, 10, 3, 3, 1, 1),     # 169 outputs (not a multiple of 4: element-wise staging), 10 channels
    (2, 1, 32, 32, 8, 3, 3, 1, 1),      # 1024 outputs: three bands of dx rows
    (2, 2, 9, 9, 12, 2, 2, 2, 0),       # stride 2, K = 8: conv_dwp
    (2, 1, 30, 30, 9, 4, 4, 1, 1),      # 16 taps
    (2, 1, 48, 48, 16, 3, 3, 1, 1),     # 2304 outputs: beyond LDS, the mask + GEMM path
    (3, 1, 27, 27, 32, 3, 3, 1, 1),     # 729 outputs, two dW chains, element-wise staging
    (2, 2, 12, 12, 20, 2, 2, 1, 0),     # Cout 20: the second chain's last 12 rows are padding
    (2, 16, 7, 7, 24, 1, 1, 1, 0),      # K = 16 from 16 input channels of a 1x1 kernel
    (2, 1, 5, 6, 3, 3, 3, 1, 2),        # padding 2: outer output rows take taps from padding only
    (2, 1, 2, 3, 5, 1, 1, 1, 0),        # 6 outputs: lane_sum's tail only
    (2, 1, 4, 4, 31, 2, 2, 1, 0),       # 9 outputs, Cout 31
    (2, 1, 20, 20, 64, 3, 3, 1, 1),     # Cout 64: conv_dwp
    (2, 1, 6, 6, 12, 3, 3, 1, 1),       # 36 outputs: lane_sum's tail of 4, one chain wave idle (Cout 12)
    (2, 16, 8, 8, 24, 1, 1, 1, 0),      # K = 16 from 16 input channels, one whole chunk of 64 outputs
    (2, 2, 9, 9, 32, 2, 2, 1, 1),       # even kernel with padding: 100 outputs, two input channels to gather
]


@pytest.mark.parametrize("case", DWP_CASES)
def test_first_layer_weight_gradient_kernel(gpu, oracle, case):
    """db and dW (and dx, fresh and accumulated) bitwise against the oracle, with and without the ReLU's flags, and
    with only some of the gradients asked for."""
    import torch

    import nnh
    N, Cin, H, W, Cout, kh, kw, s, p = case
    x = synth.mt19937_uniform(N * 37 + Cin, N * Cin * H * W).reshape(N, Cin, H, W)
    w = synth.normal(Cout + 27, (Cout, Cin, kh, kw))
    b = synth.mt19937_uniform(Cout + 28, Cout)
    for relu in (True, False):
        y, alive = nnh.conv2d_forward(dev(x), dev(w), dev(b), s, p, relu)
        _, wa = oracle.conv2d_forward(x, w, b, s, p, relu)
        gr = synth.normal(Cout + 29, tuple(y.shape))
        old = synth.normal(Cout + 30, x.shape)
        for want_dx, want_db, first in ((True, True, True), (True, True, False), (False, False, True),
                                        (False, True, True)):
            dx = (torch.full(x.shape, float("nan"), device="cuda") if first else dev(old)) if want_dx else None
            dw = torch.full(w.shape, float("nan"), device="cuda")
            db = torch.full((Cout,), float("nan"), device="cuda") if want_db else None
            nnh.conv2d_backward(dev(gr), dev(x), dev(w), alive if relu else None, s, p, dx, first, dw, True, db, True)
            wdx, wdw, wdb = oracle.conv2d_backward(gr, x, w, wa if relu else None, s, p,
                                                   dx=None if first else old, dx_first=first)
            tag = (case, relu, want_dx, want_db, first)
            same(host(dw), wdw, ("dw",) + tag)
            if want_db:
                same(host(db), wdb, ("db",) + tag)
            if want_dx:
                same(host(dx), wdx, ("dx",) + tag)


@pytest.mark.parametrize("relu", [True, False])
def test_empty_plane_with_padding(gpu, oracle, relu):
    """H = W = 0 with padding 1 and a 1x1 kernel: every output tap is padding (ho = wo = 2), so y = bias, dW is +0
    and db sums g (ops.cpp:1362 accepts the shape). The first-layer weight-gradient kernel takes this shape with no
    x to read: dW and db only (dx is empty), fresh and accumulated."""
    import ctypes as C

    import torch

    import nnh
    N, Cin, Cout = 3, 1, 5
    x = np.zeros((N, Cin, 0, 0), np.float32)
    w = synth.normal(61, (Cout, Cin, 1, 1))
    b = synth.mt19937_uniform(62, Cout, -1.0, 1.0)
    wy, wa = oracle.conv2d_forward(x, w, b, 1, 1, relu)
    xd = torch.zeros(1, device="cuda")  # a real allocation standing in for the empty plane (never read)
    y = torch.full(wy.shape, float("nan"), device="cuda")
    alive = torch.empty(wy.shape, dtype=torch.uint8, device="cuda") if relu else None
    L, P, st = nnh.lib(), nnh._ptr, nnh._stream(None)
    wd, bd = dev(w), dev(b)
    nnh.check(L.nnh_conv2d_forward(P(xd), N, Cin, 0, 0, P(wd), Cout, 1, 1, P(bd), 1, 1, int(relu), P(y), P(alive), st))
    same(host(y), wy, "y")
    gr = synth.normal(63, wy.shape)
    old_w, old_b = synth.normal(64, w.shape), synth.normal(65, (Cout,))
    for first in (True, False):
        dw = torch.full(w.shape, float("nan"), device="cuda") if first else dev(old_w)
        db = torch.full((Cout,), float("nan"), device="cuda") if first else dev(old_b)
        nnh.check(L.nnh_conv2d_backward(P(dev(gr)), P(xd), P(wd), P(alive), N, Cin, 0, 0, Cout, 1, 1, 1, 1, None,
                                        1, P(dw), int(first), P(db), int(first), st))
        _, wdw, wdb = oracle.conv2d_backward(gr, x, w, wa if relu else None, 1, 1)
        if not first:
            wdw, wdb = old_w + wdw, old_b + wdb
        same(host(dw), wdw, ("dw", relu, first))
        same(host(db), wdb, ("db", relu, first))

"""Parity of nn::matmul (Tensor batched matmul), nn::linear and the ReLU node on the GPU.

Golden vectors are nn-cpp's own outputs (tests/golden/reference_vectors.npz, written from its compiled
sources); every comparison is bitwise. BASELINE config 2 (3-layer MLP, forward and backward) is checked
against the oracle at full size.
"""
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


def same(got, want, what):
    assert_same(got, want, what)


# ------------------------------------------------------------------ matmul

def test_matmul_golden(gpu):
    import golden_cases as gc

    import nnh
    g = np.load(gc.__file__.replace("golden_cases.py", "reference_vectors.npz"))
    for name, spec in gc.MATMUL_CASES:
        a, b, ta, tb = gc.matmul_inputs(spec)
        same(host(nnh.matmul(dev(a), dev(b), ta, tb)), g[f"matmul/{name}"], name)


def test_matmul_hand_values(gpu):
    """tests/test_tensor.cpp:365-392."""
    import nnh
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    assert host(nnh.matmul(dev(a), dev(b))).tolist() == [[58, 64], [139, 154]]
    ab = np.array([1, 0, 0, 1, 2, 0, 0, 2], np.float32).reshape(2, 2, 2)
    c = host(nnh.matmul(dev(ab), dev(np.ones((2, 2, 2), np.float32))))
    assert c[0, 0, 0] == 1.0 and c[1, 0, 0] == 2.0
    import torch
    e = nnh.matmul(torch.zeros((0, 3), device="cuda"), torch.zeros((3, 2), device="cuda"))
    assert tuple(e.shape) == (0, 2)
    e = host(nnh.matmul(torch.zeros((2, 0), device="cuda"), torch.zeros((0, 3), device="cuda")))
    assert e.shape == (2, 3) and np.all(e == 0.0)
    assert tuple(nnh.matmul(torch.zeros((2, 3), device="cuda"), torch.zeros((3, 0), device="cuda")).shape) == (2, 0)


def test_matmul_flags_match_oracle(gpu, oracle):
    """test_tensor.cpp:403-442's check_flags shapes, every flag combination, bit-exact with the oracle."""
    import nnh
    from test_oracle import oracle_matmul
    rng = np.random.default_rng(1)
    for a_shape, b_shape in (((7, 33), (33, 5)), ((4, 7, 33), (4, 33, 5)), ((1, 7, 33), (4, 33, 5)),
                             ((4, 7, 33), (33, 5)), ((2, 3, 65, 129), (1, 3, 129, 70))):
        for f in range(4):
            ta, tb = bool(f & 1), bool(f & 2)
            a = rng.uniform(-1, 1, a_shape).astype(np.float32)
            b = rng.uniform(-1, 1, b_shape).astype(np.float32)
            sa = np.ascontiguousarray(np.swapaxes(a, -1, -2)) if ta else a
            sb = np.ascontiguousarray(np.swapaxes(b, -1, -2)) if tb else b
            got = host(nnh.matmul(dev(sa), dev(sb), ta, tb))
            same(got, oracle_matmul(oracle, sa, sb, ta, tb), (a_shape, b_shape, ta, tb))


def test_matmul_shape_error(gpu):
    import nnh
    with pytest.raises(nnh.ShapeError):
        import torch
        nnh.matmul(torch.zeros((2, 3), device="cuda"), torch.zeros((4, 2), device="cuda"))


# ------------------------------------------------------------------ linear

def test_linear_golden(gpu):
    import golden_cases as gc
    import torch

    import nnh
    g = np.load(gc.__file__.replace("golden_cases.py", "reference_vectors.npz"))
    for name, spec in gc.LINEAR_CASES:
        x, w, bias, gr = gc.linear_inputs(spec)
        same(host(nnh.linear_forward(dev(x), dev(w), dev(bias))), g[f"linear/{name}/y"], name)
        # nn-cpp's leaves accumulate into zero-filled gradients (first == false)
        dx, dw, db = (torch.zeros(s, device="cuda") for s in (x.shape, w.shape, bias.shape))
        nnh.linear_backward(dev(gr), dev(x), dev(w), dx, False, dw, False, db, False)
        for key, t in (("dx", dx), ("dw", dw), ("db", db)):
            same(host(t), g[f"linear/{name}/{key}"], (name, key))


def test_linear_forward_add(gpu, oracle):
    """nnh_linear_forward_add: y = residual + linear(x, w, b), bit for bit the oracle's linear and then the float
    add, on shapes each GEMM route takes (the tile kernel, the VALU kernel, the chain kernel, the pieces kernels and
    a cut of more than 16 pieces with its partials), with -0, infinities and NaN in the residual, in place (y is the
    residual), and refused when the residual overlaps y other than in place."""
    import torch

    import nnh
    cases = [(1024, 64, 64), (1024, 256, 64), (256, 32, 64), (64, 1024, 64), (33, 2048, 70), (16, 4096, 16),
             (512, 512, 512), (7, 5, 3)]
    for ci, (M, K, n) in enumerate(cases):
        x = synth.mt19937_uniform(3000 + ci, M * K).reshape(M, K)
        w = synth.mt19937_uniform(3100 + ci, n * K).reshape(n, K)
        b = synth.mt19937_uniform(3200 + ci, n)
        r = synth.normal(3300 + ci, (M, n))
        r[0, : min(n, 4)] = [-0.0, np.inf, -np.inf, np.nan][: min(n, 4)]
        want = r + oracle.linear_forward(x, w, b)
        got = nnh.linear_forward_add(dev(x), dev(w), dev(b), dev(r))
        assert_same(host(got), want, ("linear + residual", M, K, n), nan_equal=True)
        rd = dev(r)
        nnh.linear_forward_add(dev(x), dev(w), dev(b), rd, out=rd)
        assert_same(host(rd), want, ("in place", M, K, n), nan_equal=True)
    L = nnh.lib()
    buf = torch.zeros(2 * 64 * 64 + 64, device="cuda")
    x, w, b = dev(np.ones((64, 64), np.float32)), dev(np.ones((64, 64), np.float32)), dev(np.ones(64, np.float32))
    rc = L.nnh_linear_forward_add(nnh._ptr(x), 64, 64, nnh._ptr(w), 64, nnh._ptr(b), nnh._ptr(buf),
                                  nnh._ptr(buf, 64), nnh._stream(None))
    assert rc == nnh.ERR_ALIAS


def test_linear_gelu_forward(gpu, oracle):
    """nnh_linear_gelu_forward: h = linear(x, w, b) and the GELU of h (y and the kept tanh), bit for bit the oracle's
    linear and gelu, with the GELU in the chain kernel's epilogue (transformer_tiny's fc1, ragged tiles, inputs past
    tanh's clamp) and, for a product with a depth cut, as two launches; outputs that overlap are refused."""
    import torch

    import nnh
    L, P, st = nnh.lib(), nnh._ptr, nnh._stream(None)
    cases = [(1024, 64, 256), (37, 20, 70), (64, 1024, 64), (5, 3, 9)]
    for ci, (M, K, n) in enumerate(cases):
        x = synth.normal(3700 + ci, (M, K))
        w = synth.normal(3800 + ci, (n, K))
        b = synth.normal(3900 + ci, (n,))
        if ci == 1:
            b[0], b[1] = 40.0, -40.0  # outputs far past tanh's clamp of +-9
        h0 = oracle.linear_forward(x, w, b)
        y0, t0 = oracle.gelu_forward(h0)
        h, y, t = (torch.full((M, n), float("nan"), device="cuda") for _ in range(3))
        xd, wd, bd = dev(x), dev(w), dev(b)
        nnh.check(L.nnh_linear_gelu_forward(P(xd), M, K, P(wd), n, P(bd), P(h), P(y), P(t), st))
        same(host(h), h0, ("h", M, K, n))
        same(host(y), y0, ("y", M, K, n))
        same(host(t), t0, ("tanh", M, K, n))
    buf = torch.zeros(3 * 64 * 64, device="cuda")
    xd, wd, bd = dev(np.ones((64, 64), np.float32)), dev(np.ones((64, 64), np.float32)), dev(np.ones(64, np.float32))
    assert L.nnh_linear_gelu_forward(P(xd), 64, 64, P(wd), 64, P(bd), P(buf), P(buf, 64), P(buf, 8192), st) == \
        nnh.ERR_ALIAS


def test_linear_forward_multi(gpu, oracle):
    """nnh_linear_forward_multi: several linear layers over one input, each output the oracle's linear bit for bit:
    three projections of one width (one launch on the chain kernel), of different widths, with ragged tiles, a
    single layer, four layers and a depth past the group's limit (each in turn); outputs that overlap are refused."""
    import torch

    import nnh
    cases = [((16, 64, 64), [64, 64, 64]), ((100, 48), [64, 32, 16]), ((37, 20), [7, 9]), ((64, 64), [64]),
             ((64, 64), [16, 16, 16, 16]), ((64, 512), [32, 32, 32])]
    for ci, (xs, ns) in enumerate(cases):
        K = xs[-1]
        x = synth.mt19937_uniform(3400 + ci, int(np.prod(xs))).reshape(xs)
        layers = [(synth.mt19937_uniform(3500 + 10 * ci + i, n * K).reshape(n, K),
                   synth.mt19937_uniform(3600 + 10 * ci + i, n)) for i, n in enumerate(ns)]
        ys = nnh.linear_forward_multi(dev(x), [(dev(w), dev(b)) for w, b in layers])
        for i, (w, b) in enumerate(layers):
            same(host(ys[i]), oracle.linear_forward(x, w, b), (xs, ns, i))
    L = nnh.lib()
    x, w, b = dev(np.ones((64, 64), np.float32)), dev(np.ones((64, 64), np.float32)), dev(np.ones(64, np.float32))
    buf = torch.zeros(64 * 64 + 64 * 32, device="cuda")
    vp = nnh._vp
    ws = (vp * 2)(w.data_ptr(), w.data_ptr())
    bs = (vp * 2)(b.data_ptr(), b.data_ptr())
    ys = (vp * 2)(buf.data_ptr(), buf.data_ptr() + 4 * 64 * 32)
    import ctypes as C
    ns = (C.c_size_t * 2)(64, 64)
    assert L.nnh_linear_forward_multi(nnh._ptr(x), 64, 64, 2, ws, ns, bs, ys, nnh._stream(None)) == nnh.ERR_ALIAS


def test_linear_first_write_overwrites(gpu, oracle):
    """A fresh gradient is overwritten (sgemm without accumulate; bias s + 0.0f): garbage in the buffer
    must not leak into the result."""
    import torch

    import nnh
    x, w, gr = (synth.mt19937_uniform(s, n).reshape(sh) for s, n, sh in
                ((7, 300 * 70, (300, 70)), (8, 40 * 70, (40, 70)), (9, 300 * 40, (300, 40))))
    dx, dw, db = (torch.full(s, float("nan"), device="cuda") for s in (x.shape, w.shape, (40,)))
    nnh.linear_backward(dev(gr), dev(x), dev(w), dx, True, dw, True, db, True)
    want = oracle.linear_backward(gr, x, w, dx_first=True, dw_first=True, db_first=True)
    for t, wv, key in zip((dx, dw, db), want, ("dx", "dw", "db")):
        same(host(t), wv, key)


def test_linear_bias_gradient_in_weight_product(gpu, oracle):
    """db of a 2-D gradient is folded inside the dW = G^T X product (the row sums of op(A), in k order from +0);
    other cases keep the separate Tensor::sum(0). Both combines (store s + 0.0f, add to the old db), edge and
    interior tiles, several row tiles, depths that are not a multiple of the depth tile, weight gradients large
    enough for the 64 x 64 and 128 x 128 tile configurations, a product that takes nn-cpp's depth cut (db
    computed apart: 32 x 64 outputs, 1024 deep), 3-D gradients (two sums, in one launch up to 512 rows of the
    second axis: transformer_tiny's {16, 64, 64}, {35, 500, 70}; past it, {2, 513, 33}, two launches), a 4-D
    gradient (three sums), and special values in G."""
    import torch

    import nnh
    cases = [  # (batch rows M, in K, out n, leading shape)
        (300, 70, 40, None), (256, 784, 512, None), (256, 256, 10, None), (64, 128, 96, None),
        (37, 33, 129, None), (1024, 64, 32, None), (64, 1024, 1024, None), (16, 2048, 4096, None),
        (6, 50, 70, (2, 3)), (1024, 64, 64, (16, 64)), (35 * 500, 8, 70, (35, 500)), (2 * 513, 4, 33, (2, 513)),
        (60, 6, 7, (3, 4, 5)),
    ]
    for ci, (M, K, n, lead) in enumerate(cases):
        x = synth.mt19937_uniform(1000 + ci, M * K).reshape(M, K)
        w = synth.mt19937_uniform(1100 + ci, n * K).reshape(n, K)
        gr = synth.normal(1200 + ci, (M, n))
        if ci == 4:
            gr[3, 0] = np.inf
            gr[5, 1] = np.nan
            gr[:, 2] = -0.0
            gr[7, 3], gr[9, 3] = np.inf, -np.inf
        shape_x = (lead + (K,)) if lead else (M, K)
        shape_g = (lead + (n,)) if lead else (M, n)
        for first in (True, False):
            dx0 = synth.mt19937_uniform(1300 + ci, M * K).reshape(shape_x)
            dw0 = synth.mt19937_uniform(1400 + ci, n * K).reshape(n, K)
            db0 = synth.mt19937_uniform(1500 + ci, n)
            dx, dw, db = dev(dx0), dev(dw0), dev(db0)
            nnh.linear_backward(dev(gr.reshape(shape_g)), dev(x.reshape(shape_x)), dev(w), dx, first, dw, first,
                                db, first)
            want = oracle.linear_backward(gr.reshape(shape_g), x.reshape(shape_x), w, dx=dx0.copy(), dx_first=first,
                                          dw=dw0.copy(), dw_first=first, db=db0.copy(), db_first=first)
            # a NaN made by the arithmetic (inf - inf) has no defined sign bit: x86 and the GPU differ there
            for t, wv, key in zip((dx, dw, db), want, ("dx", "dw", "db")):
                assert_same(host(t), wv, (M, K, n, lead, first, key), nan_equal=(ci == 4))


def test_linear_bias_gradient_in_cut_weight_product(gpu, oracle):
    """A 3-D gradient whose weight product takes nn-cpp's depth cut runs dW on the 16x16x4 pieces kernel, and db
    (sum_to_shape's two ordered sums: over axis 0 for each index of axis 1, then over axis 1, each from +0) is
    folded into that launch: transformer_tiny's attention, fc1 and fc2 gradients ({16, 64} rows), 256 rows of the
    second axis (the most the fold takes), ragged output tiles (n = 68, 20); past the fold's limits the separate
    sums take over (257 rows of the second axis, n not a multiple of 4). Both combines, and special values in G
    (-0 columns, infinities) whose sums keep their sign; every output against the oracle, bit for bit."""
    import nnh
    cases = [  # (leading shape, in K, out n)
        ((16, 64), 64, 64), ((16, 64), 64, 256), ((16, 64), 256, 64), ((4, 256), 32, 68), ((2, 384), 80, 20),
        ((5, 257), 32, 36), ((3, 200), 64, 30),
    ]
    for ci, (lead, K, n) in enumerate(cases):
        M = lead[0] * lead[1]
        x = synth.mt19937_uniform(2000 + ci, M * K).reshape(lead + (K,))
        w = synth.mt19937_uniform(2100 + ci, n * K).reshape(n, K)
        gr = synth.normal(2200 + ci, lead + (n,))
        if ci == 3:
            gr[:, :, 1] = -0.0
            gr[1, 5, 2] = np.inf
            gr[2, 7, 3], gr[3, 9, 3] = np.inf, -np.inf
            gr[:, 3, 4] = -0.0
        for first in (True, False):
            dx0 = synth.mt19937_uniform(2300 + ci, M * K).reshape(lead + (K,))
            dw0 = synth.mt19937_uniform(2400 + ci, n * K).reshape(n, K)
            db0 = synth.mt19937_uniform(2500 + ci, n)
            if ci == 3:
                db0[1] = -0.0
            dx, dw, db = dev(dx0), dev(dw0), dev(db0)
            nnh.linear_backward(dev(gr), dev(x), dev(w), dx, first, dw, first, db, first)
            want = oracle.linear_backward(gr, x, w, dx=dx0.copy(), dx_first=first, dw=dw0.copy(), dw_first=first,
                                          db=db0.copy(), db_first=first)
            for t, wv, key in zip((dx, dw, db), want, ("dx", "dw", "db")):
                assert_same(host(t), wv, (lead, K, n, first, key), nan_equal=(ci == 3))


def test_linear_backward_dx_dw_in_one_launch(gpu, oracle):
    """dX = G W and dW = G^T X of one Linear run in one launch when both pick the same small-tile configuration
    (4x4x1 and 16x16x1 tiles, interior and edge, with and without db inside dW). Buffers that overlap keep the
    reference's order, dX then dW: dx overlapping dw ends with dW's values where they meet, and dx on x itself
    makes dW read the new dX."""
    import torch

    import nnh
    cases = [(256, 784, 512), (256, 512, 256), (256, 256, 10), (1024, 1024, 1024), (96, 64, 64)]
    for ci, (M, K, n) in enumerate(cases):
        x = synth.mt19937_uniform(1600 + ci, M * K).reshape(M, K)
        w = synth.mt19937_uniform(1700 + ci, n * K).reshape(n, K)
        gr = synth.normal(1800 + ci, (M, n))
        for first, with_db in ((True, True), (False, True), (False, False)):
            dx0 = synth.mt19937_uniform(1900 + ci, M * K).reshape(M, K)
            dw0 = synth.mt19937_uniform(2000 + ci, n * K).reshape(n, K)
            db0 = synth.mt19937_uniform(2100 + ci, n)
            dx, dw = dev(dx0), dev(dw0)
            db = dev(db0) if with_db else None
            nnh.linear_backward(dev(gr), dev(x), dev(w), dx, first, dw, first, db, first)
            want = oracle.linear_backward(gr, x, w, dx=dx0.copy(), dx_first=first, dw=dw0.copy(), dw_first=first,
                                          db=db0.copy(), db_first=first)
            for t, wv, key in zip((dx, dw, db), want, ("dx", "dw", "db")):
                if t is not None:
                    same(host(t), wv, (M, K, n, first, with_db, key))
    # overlapping buffers: one allocation holds dx, and dw starts inside it
    M, K, n = 256, 512, 256
    x = synth.mt19937_uniform(2200, M * K).reshape(M, K)
    w = synth.mt19937_uniform(2201, n * K).reshape(n, K)
    gr = synth.normal(2202, (M, n))
    want_dx, want_dw, _ = oracle.linear_backward(gr, x, w, dx_first=True, dw_first=True, db_first=True)
    buf = torch.zeros(M * K + n * K // 2, device="cuda")
    dx, dw = buf[:M * K].view(M, K), buf[M * K - n * K // 2:].view(n, K)
    nnh.linear_backward(dev(gr), dev(x), dev(w), dx, True, dw, True, None, True)
    mem = np.zeros(M * K + n * K // 2, np.float32)
    mem[:M * K] = want_dx.ravel()
    mem[M * K - n * K // 2:] = want_dw.ravel()
    same(host(buf), mem, "dx overlapped by dw")
    # dx is x: dW = G^T (new dX)
    xd = dev(x)
    dw = torch.zeros((n, K), device="cuda")
    nnh.linear_backward(dev(gr), xd, dev(w), xd, True, dw, True, None, True)
    new_x = want_dx
    _, want_dw2, _ = oracle.linear_backward(gr, new_x, w, dx_first=True, dw_first=True, db_first=True)
    same(host(xd), want_dx, "dx written over x")
    same(host(dw), want_dw2, "dw from the new x")


def test_relu_node(gpu, oracle):
    import torch

    import nnh
    x = synth.mt19937_uniform(5, 10007)
    x[::97] = 0.0
    x[1::101] = -0.0
    y = host(nnh.relu_forward(dev(x)))
    same(y, oracle.relu(x), "relu forward")
    g = synth.mt19937_uniform(6, 10007)
    for first in (True, False):
        d0 = synth.mt19937_uniform(7, 10007)
        d = dev(d0)
        nnh.relu_backward(dev(x), dev(g), d, first)
        term = np.where(x > 0, g, np.float32(0)).astype(np.float32)
        want = (term + np.float32(0)) if first else (d0 + term)
        same(host(d), want.astype(np.float32), f"relu backward first={first}")


def test_baseline_config2_mlp(gpu, oracle):
    """X[256 x 784] ~ U[0,1], layers 784->512->256->10 with weights {out, in} ~ U(+-1/sqrt(in))
    (nn-cpp's Linear init bound), zero biases, y = ReLU(X W^T + b) per layer; backward of each layer with
    dY ~ N(0,1): dX = dY W, dW = dY^T X, db. Everything bit-identical to nn-cpp's arithmetic."""
    import torch

    import nnh
    dims = [784, 512, 256, 10]
    x = synth.mt19937_uniform(1, 256 * 784, 0.0, 1.0).reshape(256, 784)
    acts = [x]
    for li in range(3):
        fan_in, fan_out = dims[li], dims[li + 1]
        bound = float(1.0 / np.sqrt(fan_in))
        w = synth.mt19937_uniform(100 + li, fan_out * fan_in, -bound, bound).reshape(fan_out, fan_in)
        b = np.zeros(fan_out, np.float32)
        y_gpu = host(nnh.linear_forward(dev(acts[-1]), dev(w), dev(b), relu=True))
        y_ref = oracle.relu(oracle.linear_forward(acts[-1], w, b))
        same(y_gpu, y_ref, f"layer {li} forward")
        gy = synth.normal(200 + li, (256, fan_out))
        dx, dw, db = (torch.zeros(s, device="cuda") for s in ((256, fan_in), w.shape, b.shape))
        nnh.linear_backward(dev(gy), dev(acts[-1]), dev(w), dx, True, dw, True, db, True)
        want = oracle.linear_backward(gy, acts[-1], w, dx_first=True, dw_first=True, db_first=True)
        for t, wv, key in zip((dx, dw, db), want, ("dx", "dw", "db")):
            same(host(t), wv, f"layer {li} {key}")
        acts.append(y_ref)


def test_tensor_sum0_every_shape_and_combine(gpu, oracle):
    """Tensor::sum(0) (src/tensor.cpp:422-456): rows added in order from +0. Row counts around the kernel's
    128-row chunks, widths that are not multiples of 4 or of its 32-column blocks (36 and 100: a last block whose
    width is a multiple of 4 below 32, where the 16-byte path clamps its last group), an unaligned source (the
    4-byte path), and the three combines: store, store s + 0.0f (a fresh gradient: -0 becomes +0), add."""
    import torch

    import nnh
    seed = 900
    for rows in (0, 1, 7, 127, 128, 129, 300):
        for inner in (1, 3, 10, 36, 64, 65, 100, 130, 512):
            src = synth.mt19937_uniform(seed, max(rows * inner, 1), -1.0, 1.0)[: rows * inner].reshape(rows, inner)
            seed += 1
            if rows:
                src[0, 0] = -0.0  # a one-row column sum of -0 is -0 stored, +0 with combine 1
            base = synth.mt19937_uniform(seed, inner, -1.0, 1.0)
            s = oracle.sum_axis0(src) if rows else np.zeros(inner, np.float32)
            for offset in (0, 1):
                buf = torch.zeros(rows * inner + offset + 1, device="cuda")
                view = buf[offset: offset + rows * inner]
                view.copy_(torch.from_numpy(src.reshape(-1)))
                for combine, want in ((0, s), (1, s + np.float32(0.0)), (2, base + s)):
                    dst = torch.from_numpy(base.copy()).cuda()
                    nnh.tensor_sum0(view.reshape(rows, inner) if rows else view.reshape(0, inner), dst, combine)
                    same(host(dst), want.astype(np.float32), (rows, inner, offset, combine))

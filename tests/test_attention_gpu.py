"""Parity of nn::attention (forward and backward) and nn::scaled_masked_softmax on the GPU.

Every step is bit-identical to nn-cpp: the GEMMs (QK^T, PV and the four backward products), the scale, the
masks, the max scan, the exp (the GPU restates glibc's expf, which nn-cpp's std::exp(float) calls), the in-order
row sum, the division and the softmax backward. So every comparison is bitwise: against the oracle (which calls
glibc's expf) at every shape, and against nn-cpp's own outputs (golden vectors).
Shapes: the reference's test cases and BASELINE config 4 (32 x 8 heads x 256 x 64, and its causal variant).
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


def golden():
    import golden_cases as gc
    return gc, np.load(gc.__file__.replace("golden_cases.py", "reference_vectors.npz"))


def test_attention_golden_forward_backward(gpu, oracle):
    import torch

    import nnh
    gc, g = golden()
    for name, spec in gc.ATTENTION_CASES:
        q, k, v, heads, mask, causal, gr = gc.attention_inputs(spec)
        out, probs = nnh.attention_forward(dev(q), dev(k), dev(v), heads, dev(mask), causal)
        # nn-cpp's leaves accumulate into zero-filled gradients (first == false)
        dq, dk, dv = (torch.zeros(t.shape, device="cuda") for t in (q, k, v))
        nnh.attention_backward(dev(gr), dev(q), dev(k), dev(v), probs, heads, dev(mask), causal, dq, False, dk, False,
                               dv, False)
        wo, wp = oracle.attention_forward(q, k, v, heads, mask, causal)
        wq, wk, wv = oracle.attention_backward(gr, q, k, v, wp, heads, mask, causal)
        same(host(out), wo, (name, "out"))
        same(host(probs), wp, (name, "probs"))
        same(host(out), g[f"attention/{name}/out"], (name, "out vs nn-cpp"))
        for key, t, w in (("dq", dq, wq), ("dk", dk, wk), ("dv", dv, wv)):
            same(host(t), w, (name, key))
            same(host(t), g[f"attention/{name}/{key}"], (name, key, "vs nn-cpp"))


def composed(q, k, v, heads, mask, causal):
    """test_autograd.cpp:1533-1540: split heads, matmul_bt, scaled_masked_softmax, matmul, merge heads,
    every step through this library."""
    import nnh
    N, Tq, D = q.shape
    Tk = k.shape[1]
    Dh = D // heads

    def split(x, T):
        return x.reshape(N, T, heads, Dh).transpose(1, 2).contiguous()

    s = nnh.matmul(split(q, Tq), split(k, Tk), False, True)
    w = nnh.scaled_masked_softmax_forward(s, np.float32(1.0) / np.sqrt(np.float32(Dh)), mask, causal)
    o = nnh.matmul(w, split(v, Tk))
    return o.transpose(1, 2).contiguous().reshape(N, Tq, D), w


def test_attention_gives_the_bits_of_the_composed_ops(gpu):
    """test_autograd.cpp:1597-1620 on this backend: the fused op equals the composition of matmul_bt,
    scaled_masked_softmax and matmul, bit for bit (the per-element depth order never depends on the caller)."""
    import nnh
    mask = np.array([[1, 1, 1, 1, 0], [1, 1, 1, 1, 1], [1, 1, 0, 0, 0]], np.float32)
    for tq, tk, causal, padded in ((5, 5, True, False), (5, 5, True, True), (4, 5, False, True), (5, 5, False, False)):
        q = dev(synth.mt19937_uniform(1, 3 * tq * 8).reshape(3, tq, 8))
        k = dev(synth.mt19937_uniform(2, 3 * tk * 8).reshape(3, tk, 8))
        v = dev(synth.mt19937_uniform(3, 3 * tk * 8).reshape(3, tk, 8))
        m = dev(mask) if padded else None
        out, probs = nnh.attention_forward(q, k, v, 4, m, causal)
        co, cw = composed(q, k, v, 4, m, causal)
        same(host(out), host(co), (tq, tk, causal, padded))
        same(host(probs), host(cw), ("probs", tq, tk, causal, padded))


@pytest.mark.parametrize("causal", [False, True])
def test_baseline_config4(gpu, oracle, causal):
    """batch 32, 8 heads, seq 256, head_dim 64, Q, K, V ~ N(0, 1) (seed 3); scale 1/8.
    Probabilities and output bitwise equal to the oracle's; causal rows hold exact zeros past the diagonal."""
    import nnh
    N, T, D, H = 32, 256, 512, 8
    q, k, v = (synth.normal(3 + i, (N, T, D)) for i in range(3))
    out, probs = nnh.attention_forward(dev(q), dev(k), dev(v), H, None, causal)
    out, probs = host(out), host(probs)
    ref_out, ref_probs = oracle.attention_forward(q, k, v, H, None, causal)
    same(probs, ref_probs, "probs")
    same(out, ref_out, "out")
    if causal:
        tri = np.triu(np.ones((T, T), bool), 1)
        assert np.all(probs[:, :, tri] == 0.0)


# Head width 64, Tk <= 256, Tk % 4 == 0: the fused forward kernel (one workgroup per 64 query rows). Ragged query
# blocks, key counts that do not fill a wave's 64 keys, causal rows, padded keys.
FUSED_SHAPES = [  # (N, Tq, Tk, heads, causal, masked)
    (2, 1, 4, 1, False, False),
    (2, 37, 36, 2, False, True),
    (1, 64, 64, 1, True, False),
    (2, 100, 100, 2, True, True),
    (1, 130, 252, 3, False, True),
    (2, 256, 256, 2, True, True),
    # Tk a multiple of 16: O = P V on 16x16x4 (ragged and whole 64-row blocks, key counts that are not a multiple of
    # 64)
    (2, 48, 160, 2, False, True),
    (1, 16, 16, 1, True, False),
    (1, 112, 240, 1, False, False),
]
# The three-launch path: key count not a multiple of 4, more than 256 keys, head width 32.
UNFUSED_SHAPES = [  # (N, Tq, Tk, heads, Dh, causal, masked)
    (2, 50, 37, 2, 64, False, True),
    (1, 40, 260, 1, 64, False, False),
    (2, 70, 70, 4, 32, True, True),
]


def attention_case(seed, N, Tq, Tk, D, masked):
    q = synth.normal(seed, (N, Tq, D))
    k = synth.normal(seed + 1, (N, Tk, D))
    v = synth.normal(seed + 2, (N, Tk, D))
    mask = None
    if masked:
        mask = np.ones((N, Tk), np.float32)
        mask[0, Tk // 2:] = 0
        if N > 1:
            mask[1, ::3] = 0
    return q, k, v, mask


@pytest.mark.parametrize("shape", FUSED_SHAPES)
def test_fused_forward_matches_oracle(gpu, oracle, shape):
    import nnh
    N, Tq, Tk, H, causal, masked = shape
    q, k, v, mask = attention_case(60 + Tq, N, Tq, Tk, 64 * H, masked)
    out, probs = nnh.attention_forward(dev(q), dev(k), dev(v), H, dev(mask), causal)
    want_out, want_probs = oracle.attention_forward(q, k, v, H, mask, causal)
    same(host(probs), want_probs, (shape, "probs"))
    same(host(out), want_out, (shape, "out"))


@pytest.mark.parametrize("shape", UNFUSED_SHAPES)
def test_unfused_forward_matches_oracle(gpu, oracle, shape):
    import nnh
    N, Tq, Tk, H, Dh, causal, masked = shape
    q, k, v, mask = attention_case(80 + Tq, N, Tq, Tk, Dh * H, masked)
    out, probs = nnh.attention_forward(dev(q), dev(k), dev(v), H, dev(mask), causal)
    want_out, want_probs = oracle.attention_forward(q, k, v, H, mask, causal)
    same(host(probs), want_probs, (shape, "probs"))
    same(host(out), want_out, (shape, "out"))


def backward_case(oracle, q, k, v, mask, H, causal, seed):
    """dQ, dK, dV from the library (fresh gradients) and from the oracle, for upstream gradient N(0, 1)."""
    import torch

    import nnh
    g = synth.normal(seed, q.shape)
    _, probs = oracle.attention_forward(q, k, v, H, mask, causal)
    dq, dk, dv = (torch.full(t.shape, float("nan"), device="cuda") for t in (q, k, v))
    nnh.attention_backward(dev(g), dev(q), dev(k), dev(v), dev(probs), H, dev(mask), causal, dq, True, dk, True, dv,
                           True)
    want = oracle.attention_backward(g, q, k, v, probs, H, mask, causal)
    return (host(dq), host(dk), host(dv)), want


@pytest.mark.parametrize("shape", FUSED_SHAPES)
def test_fused_backward_matches_oracle(gpu, oracle, shape):
    """The fused dP + softmax backward kernel (same shapes as the fused forward), then dQ, dK, dV."""
    N, Tq, Tk, H, causal, masked = shape
    q, k, v, mask = attention_case(70 + Tq, N, Tq, Tk, 64 * H, masked)
    got, want = backward_case(oracle, q, k, v, mask, H, causal, 75 + Tq)
    for t, w, key in zip(got, want, ("dq", "dk", "dv")):
        same(t, w, (shape, key))


@pytest.mark.parametrize("shape", UNFUSED_SHAPES)
def test_unfused_backward_matches_oracle(gpu, oracle, shape):
    N, Tq, Tk, H, Dh, causal, masked = shape
    q, k, v, mask = attention_case(85 + Tq, N, Tq, Tk, Dh * H, masked)
    got, want = backward_case(oracle, q, k, v, mask, H, causal, 87 + Tq)
    for t, w, key in zip(got, want, ("dq", "dk", "dv")):
        same(t, w, (shape, key))


def test_fused_forward_special_values(gpu, oracle):
    """Inf and NaN in Q, K and V: the fused kernels' chains, max scan, division and softmax backward propagate them
    as nn-cpp does (NaN payloads aside)."""
    import nnh
    N, T, H = 2, 96, 2
    q, k, v, _ = attention_case(90, N, T, T, 64 * H, False)
    q[0, 3, 5] = np.inf
    k[0, 7, 70] = -np.inf
    k[1, 0, 1] = np.nan
    v[0, 11, 2] = np.nan
    v[1, 50, 64] = np.inf
    for causal in (False, True):
        out, probs = nnh.attention_forward(dev(q), dev(k), dev(v), H, None, causal)
        want_out, want_probs = oracle.attention_forward(q, k, v, H, None, causal)
        assert_same(host(probs), want_probs, ("probs", causal), nan_equal=True)
        assert_same(host(out), want_out, ("out", causal), nan_equal=True)
        got, want = backward_case(oracle, q, k, v, None, H, causal, 95)
        for t, w, key in zip(got, want, ("dq", "dk", "dv")):
            assert_same(t, w, (key, causal), nan_equal=True)


def division_rows(T):
    """Score rows [0, 0, 0, 0, 0, 0, x, -1e4]: six keys at the maximum, so the sum is 6 and p_6 / 6 for x in the
    subnormal range of exp hits exact midpoints between subnormal floats (p = 3 M 2^-149 with M odd)."""
    x = np.linspace(-103.9, -87.4, T, dtype=np.float32)
    rows = np.zeros((T, 8), np.float32)
    rows[:, 6] = x
    rows[:, 7] = -1e4
    return rows


def test_softmax_division_at_subnormal_midpoints(gpu, oracle):
    """Both softmax kernels (the fused attention and the row softmax) against the oracle's float division on rows
    whose quotients are subnormal, some exactly halfway between two floats."""
    import nnh
    T, H = 4096, 1
    rows = division_rows(T)
    y = nnh.scaled_masked_softmax_forward(dev(rows.reshape(1, 1, T, 8)), 1.0, None, False)
    assert_same(host(y), oracle.scaled_masked_softmax(rows.reshape(1, 1, T, 8), np.float32(1.0), None, False),
                "row softmax")
    # attention with S = Q K^T equal to 8 * rows: q_i = [1, 8 x_i, 0...], k_j picks a column (scale 1/8)
    N, Tq = T // 256, 256
    q = np.zeros((N, Tq, 64), np.float32)
    q[..., 0] = 1
    q[..., 1] = (8 * rows[:, 6]).reshape(N, Tq)
    k = np.zeros((N, 8, 64), np.float32)
    k[:, 6, 1] = 1
    k[:, 7, 0] = -8e4
    v = synth.normal(5, (N, 8, 64))
    out, probs = nnh.attention_forward(dev(q), dev(k), dev(v), H, None, False)
    want_out, want_probs = oracle.attention_forward(q, k, v, H, None, False)
    assert (want_probs[..., 6] < 2 ** -126).all() and (want_probs[..., 6] > 0).any()
    same(host(probs), want_probs, "attention probs")
    same(host(out), want_out, "attention out")


def test_attention_backward_matches_oracle(gpu, oracle):
    import torch

    import nnh
    N, T, D, H = 4, 256, 512, 8
    q, k, v, g = (synth.normal(30 + i, (N, T, D)) for i in range(4))
    mask = np.ones((N, T), np.float32)
    mask[1, 200:] = 0
    for causal in (False, True):
        out, probs = nnh.attention_forward(dev(q), dev(k), dev(v), H, dev(mask), causal)
        dq, dk, dv = (torch.full((N, T, D), float("nan"), device="cuda") for _ in range(3))
        nnh.attention_backward(dev(g), dev(q), dev(k), dev(v), probs, H, dev(mask), causal, dq, True, dk, True, dv,
                               True)
        _, want_probs = oracle.attention_forward(q, k, v, H, mask, causal)
        same(host(probs), want_probs, ("probs", causal))
        want = oracle.attention_backward(g, q, k, v, want_probs, H, mask, causal)
        for t, w, key in zip((dq, dk, dv), want, ("dq", "dk", "dv")):
            same(host(t), w, (key, causal))


def test_self_attention_gradient_sums_the_three_roles(gpu, oracle):
    """One node as query, key and value (test_autograd.cpp:1591-1594): dV is stored first, dQ and dK add."""
    import nnh
    x = synth.mt19937_uniform(44, 2 * 7 * 12).reshape(2, 7, 12)
    g = synth.mt19937_uniform(45, 2 * 7 * 12).reshape(2, 7, 12)
    dx_, gx = dev(x), dev(g)
    out, probs = nnh.attention_forward(dx_, dx_, dx_, 3, None, True)
    grad = dev(np.full(x.shape, np.nan, np.float32))
    nnh.attention_backward(gx, dx_, dx_, dx_, probs, 3, None, True, grad, False, grad, False, grad, True)
    want = np.zeros_like(x)
    L = oracle.lib
    from pyoracle import _fp
    _, p = oracle.attention_forward(x, x, x, 3, None, True)
    L.oracle_attention_backward(_fp(g), _fp(x), _fp(x), _fp(x), _fp(p), 2, 7, 7, 12, 3, None, 1, _fp(want), 0,
                                _fp(want), 0, _fp(want), 1)
    same(host(grad), want, "self-attention gradient")


def test_head64_dq_dk_accumulate_subsets_and_one_node(gpu, oracle):
    """dQ and dK of head width 64 after the fused dS kernel: accumulating into old gradients, with only one of the
    two asked for, and with q, k and v one node (dV stored first, then dQ and dK added: the reference's order),
    over ragged 64-row blocks, padded keys and causal rows."""
    import nnh
    from pyoracle import _fp
    L = oracle.lib
    N, T, H = 2, 100, 2
    D = 64 * H
    q, k, v, mask = attention_case(120, N, T, T, D, True)
    g = synth.normal(125, (N, T, D))
    for causal in (False, True):
        _, p = oracle.attention_forward(q, k, v, H, mask, causal)
        for want_dq, want_dk in ((True, True), (True, False), (False, True)):
            dq0, dk0 = synth.normal(126, q.shape), synth.normal(127, k.shape)
            dq, dk = (dev(dq0) if want_dq else None), (dev(dk0) if want_dk else None)
            nnh.attention_backward(dev(g), dev(q), dev(k), dev(v), dev(p), H, dev(mask), causal, dq, False, dk, False,
                                   None, True)
            wq, wk = dq0.copy(), dk0.copy()
            L.oracle_attention_backward(_fp(g), _fp(q), _fp(k), _fp(v), _fp(p), N, T, T, D, H, _fp(mask), int(causal),
                                        _fp(wq) if want_dq else None, 0, _fp(wk) if want_dk else None, 0, None, 1)
            if want_dq:
                same(host(dq), wq, (causal, "dq accumulated"))
            if want_dk:
                same(host(dk), wk, (causal, "dk accumulated"))
        # one node: x is query, key and value
        x = q
        _, px = oracle.attention_forward(x, x, x, H, mask, causal)
        for dv_first, dq_first, dk_first in ((True, False, False), (False, False, False), (False, True, False)):
            old = synth.normal(128, x.shape)
            grad = dev(old)
            nnh.attention_backward(dev(g), dev(x), dev(x), dev(x), dev(px), H, dev(mask), causal, grad, dq_first, grad,
                                   dk_first, grad, dv_first)
            want = old.copy()
            L.oracle_attention_backward(_fp(g), _fp(x), _fp(x), _fp(x), _fp(px), N, T, T, D, H, _fp(mask), int(causal),
                                        _fp(want), int(dq_first), _fp(want), int(dk_first), _fp(want), int(dv_first))
            same(host(grad), want, (causal, dv_first, dq_first, dk_first, "one node"))


def test_head64_dq_dk_accumulate_whole_blocks(gpu, oracle):
    """dQ and dK of head width 64 with Tq and Tk multiples of 16 (whole 16-row tiles): added to old gradients and
    stored fresh, causal and padded, against the oracle."""
    import nnh
    from pyoracle import _fp
    L = oracle.lib
    N, T, H = 2, 96, 2
    D = 64 * H
    q, k, v, mask = attention_case(130, N, T, T, D, True)
    g = synth.normal(135, (N, T, D))
    for causal in (False, True):
        _, p = oracle.attention_forward(q, k, v, H, mask, causal)
        for first in (False, True):
            dq0, dk0 = synth.normal(136, q.shape), synth.normal(137, k.shape)
            dq, dk = dev(dq0), dev(dk0)
            nnh.attention_backward(dev(g), dev(q), dev(k), dev(v), dev(p), H, dev(mask), causal, dq, first, dk, first,
                                   None, True)
            wq, wk = dq0.copy(), dk0.copy()
            L.oracle_attention_backward(_fp(g), _fp(q), _fp(k), _fp(v), _fp(p), N, T, T, D, H, _fp(mask), int(causal),
                                        _fp(wq), int(first), _fp(wk), int(first), None, 1)
            same(host(dq), wq, (causal, first, "dq"))
            same(host(dk), wk, (causal, first, "dk"))


def test_attention_hand_reference_and_masks(gpu):
    """test_transformer.cpp:149-176 (one head, identity projections) and 232-276 (a fully masked row is
    finite: exactly the mean of V)."""
    import nnh
    x = np.array([1, 0, 0, 2], np.float32).reshape(1, 2, 2)
    out, _ = nnh.attention_forward(dev(x), dev(x), dev(x), 1)
    out = host(out)
    s = np.float32(np.sqrt(2.0))
    for i in range(2):
        s0 = (x[0, i, 0] * x[0, 0, 0] + x[0, i, 1] * x[0, 0, 1]) / s
        s1 = (x[0, i, 0] * x[0, 1, 0] + x[0, i, 1] * x[0, 1, 1]) / s
        e0, e1 = np.exp(s0), np.exp(s1)
        for c in range(2):
            want = (e0 * x[0, 0, c] + e1 * x[0, 1, c]) / (e0 + e1)
            assert abs(out[0, i, c] - want) <= 1e-5 * abs(want) + 1e-7
    xs = synth.mt19937_uniform(3, 32).reshape(2, 4, 4)
    none = np.array([[0, 0, 0, 0], [1, 1, 1, 1]], np.float32)
    o, _ = nnh.attention_forward(dev(xs), dev(xs), dev(xs), 2, dev(none), False)
    o = host(o)
    assert np.all(np.isfinite(o))
    assert np.allclose(o[0], np.broadcast_to(xs[0].mean(axis=0), (4, 4)), rtol=1e-5, atol=1e-6)


def test_scaled_masked_softmax_matches_oracle(gpu, oracle):
    import nnh
    x = synth.normal(9, (2, 3, 33, 40))
    mask = np.ones((2, 40), np.float32)
    mask[0, 35:] = 0
    for causal, m in ((False, None), (False, mask), (True, None)):
        if causal:
            x = synth.normal(10, (2, 3, 40, 40))
        y = nnh.scaled_masked_softmax_forward(dev(x), 0.3, dev(m), causal)
        same(host(y), oracle.scaled_masked_softmax(x, np.float32(0.3), m, causal), ("forward", causal))
    x = synth.normal(11, (2, 3, 17, 17))
    y = oracle.scaled_masked_softmax(x, np.float32(0.5), None, True)
    gr = synth.normal(12, y.shape)
    for first in (True, False):
        d0 = synth.normal(13, y.shape)
        d = dev(d0)
        nnh.scaled_masked_softmax_backward(dev(y), dev(gr), d, 0.5, None, True, first)
        want = oracle.scaled_masked_softmax_backward(y, gr, np.float32(0.5), None, True, dx=d0, first=first)
        same(host(d), want, ("backward", first))


def test_softmax_exp_is_glibc_expf_over_its_whole_range(gpu, oracle):
    """Rows [x, 0] with scale 1 give p_0 = e^x / (e^x + 1) with the max 0, so the row softmax sees exp at x. x runs
    over every 61st float in [-104, 0] (about 18 million values: normal, subnormal and underflowing results),
    plus -inf, NaN, -0 and the glibc edge cases; the outputs must be the oracle's, which calls glibc's expf."""
    import nnh
    lo, hi = np.uint32(0x80000000), np.uint32(0xc2d00000)  # -0 .. -104
    bits = np.arange(lo, hi, 61, dtype=np.uint32)
    specials = np.array([0xff800000, 0x7fc00000, 0x80000000, 0xc2cff1b4, 0xc2cff1b5, 0xc2aeac50, 0xc2aeac4f,
                         0xc2b00000, 0xbf800000], np.uint32)
    x = np.concatenate([bits, specials]).view(np.float32)
    rows = np.stack([x, np.zeros_like(x)], axis=1).reshape(1, 1, -1, 2)
    y = nnh.scaled_masked_softmax_forward(dev(rows), 1.0, None, False)
    assert_same(host(y), oracle.scaled_masked_softmax(rows, np.float32(1.0), None, False), "softmax of [x, 0]",
                nan_equal=True)


def test_attention_shape_errors(gpu):
    """test_autograd.cpp:1634-1640: heads must divide D; causal needs Tq == Tk."""
    import torch

    import nnh
    q = torch.zeros((2, 4, 6), device="cuda")
    with pytest.raises(nnh.ShapeError):
        nnh.attention_forward(q, q, q, 4)
    k5 = torch.zeros((2, 5, 6), device="cuda")
    with pytest.raises(nnh.ShapeError):
        nnh.attention_forward(q, k5, k5, 2, None, True)

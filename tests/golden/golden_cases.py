"""Case definitions of the golden vectors: each case's inputs come from its seed through the reference's
own uniform stream (nnh.synth.mt19937_uniform), so only outputs are stored in reference_vectors.npz."""
import numpy as np

from nnh import synth

SENTINEL = np.float32(1e30)

# name, (trans_a, trans_b, m, n, k, accumulate, ld pad, seed)
SGEMM_CASES = [
    ("nn_7x33x17", (0, 0, 7, 33, 17, 0, 0, 11)),
    ("tn_33x7x257_acc", (1, 0, 33, 7, 257, 1, 0, 12)),
    ("nt_40x48x589_cut_pad3", (0, 1, 40, 48, 589, 0, 3, 13)),
    ("tt_64x64x1024_cut_acc", (1, 1, 64, 64, 1024, 1, 0, 14)),
    ("nn_129x65x300_acc_pad1", (0, 0, 129, 65, 300, 1, 1, 15)),
    ("tt_5x9x1100_cut_pad2", (1, 1, 5, 9, 1100, 0, 2, 16)),
    ("nt_101x75x300_pad2", (0, 1, 101, 75, 300, 0, 2, 17)),
    ("tn_64x64x511_acc", (1, 0, 64, 64, 511, 1, 0, 18)),
    ("nn_1x1x1", (0, 0, 1, 1, 1, 0, 0, 19)),
    ("nn_3x5x0_acc", (0, 0, 3, 5, 0, 1, 0, 20)),
    ("nn_3x5x0", (0, 0, 3, 5, 0, 0, 0, 21)),
]


def _stored(vals, rows, cols, ld):
    out = np.full((max(rows, 1), max(ld, 1)), SENTINEL, np.float32)
    if rows and cols:
        out[:rows, :cols] = vals.reshape(rows, cols)
    return np.ascontiguousarray(out)


def sgemm_inputs(ta, tb, m, n, k, acc, pad, seed):
    a_rows, a_cols = (k, m) if ta else (m, k)
    b_rows, b_cols = (n, k) if tb else (k, n)
    lda, ldb, ldc = a_cols + pad, b_cols + pad, n + pad
    sa, sb, sc = a_rows * a_cols, b_rows * b_cols, m * n
    v = synth.mt19937_uniform(seed, sa + sb + sc)
    return (_stored(v[:sa], a_rows, a_cols, lda), lda, _stored(v[sa:sa + sb], b_rows, b_cols, ldb), ldb,
            _stored(v[sa + sb:], m, n, ldc), ldc)


# name, (a shape, b shape, trans_a, trans_b, seed)
MATMUL_CASES = [
    ("plain_7x33_33x5", ((7, 33), (33, 5), 0, 0, 31)),
    ("batched_4x7x33_4x33x5", ((4, 7, 33), (4, 33, 5), 0, 0, 32)),
    ("broadcast_1x7x33_4x33x5", ((1, 7, 33), (4, 33, 5), 0, 0, 33)),
    ("fold_4x7x33_33x5", ((4, 7, 33), (33, 5), 0, 0, 34)),
    ("tn_batched_3x33x7_3x33x5", ((3, 33, 7), (3, 33, 5), 1, 0, 35)),
    ("nt_fold_2x3x7x33_5x33", ((2, 3, 7, 33), (5, 33), 0, 1, 36)),
    ("broadcast4d_2x1x7x9_1x3x9x6_tt", ((2, 1, 9, 7), (1, 3, 6, 9), 1, 1, 37)),
    ("depthcut_batch_2x64x600_2x600x64", ((2, 64, 600), (2, 600, 64), 0, 0, 38)),
]


def matmul_inputs(spec):
    ash, bsh, ta, tb, seed = spec
    a, b = synth.uniform_operands(seed, [ash, bsh])
    return np.ascontiguousarray(a), np.ascontiguousarray(b), ta, tb


# name, (x shape, out features, seed)
LINEAR_CASES = [
    ("2d_7x5_to_9", ((7, 5), 9, 41)),
    ("3d_3x6x5_to_9", ((3, 6, 5), 9, 42)),
    ("2d_64x600_to_40_cut", ((64, 600), 40, 43)),
    ("2d_1100x48_to_40_cut", ((1100, 48), 40, 44)),
]


def linear_inputs(spec):
    xs, n, seed = spec
    K = xs[-1]
    ys = tuple(xs[:-1]) + (n,)
    x, w, bias, g = synth.uniform_operands(seed, [xs, (n, K), (n,), ys])
    return tuple(np.ascontiguousarray(t) for t in (x, w, bias, g))


# name, (N, Cin, H, W, Cout, ksize, stride, pad, fuse_relu, seed)
CONV_CASES = [
    ("b7_2x9x6_to3_k3s2p1", (7, 2, 9, 6, 3, 3, 2, 1, 0, 51)),
    ("b7_2x9x6_to3_k3s2p1_relu", (7, 2, 9, 6, 3, 3, 2, 1, 1, 52)),
    ("b3_2x33x5_to2_k4s3p3_relu", (3, 2, 33, 5, 2, 4, 3, 3, 1, 53)),
    ("b4_3x16x16_to4_k3s1p1_relu", (4, 3, 16, 16, 4, 3, 1, 1, 1, 54)),
    ("b2_1x2x2_to2_k5s1p2", (2, 1, 2, 2, 2, 5, 1, 2, 0, 55)),
]


def conv_inputs(spec):
    N, Cin, H, W, Cout, kk, stride, pad, relu, seed = spec
    ho, wo = (H + 2 * pad - kk) // stride + 1, (W + 2 * pad - kk) // stride + 1
    x, w, bias, g = synth.uniform_operands(seed, [(N, Cin, H, W), (Cout, Cin, kk, kk), (Cout,), (N, Cout, ho, wo)])
    return (np.ascontiguousarray(x), np.ascontiguousarray(w), np.ascontiguousarray(bias), np.ascontiguousarray(g),
            stride, pad, relu)


# name, (N, Tq, Tk, D, heads, padded, causal, seed)
ATTENTION_CASES = [
    ("n3_t5_d8_h4", (3, 5, 5, 8, 4, 0, 0, 61)),
    ("n3_t5_d8_h4_causal", (3, 5, 5, 8, 4, 0, 1, 62)),
    ("n3_t5_d8_h4_causal_pad", (3, 5, 5, 8, 4, 1, 1, 63)),
    ("n3_tq4_tk5_d8_h4_pad", (3, 4, 5, 8, 4, 1, 0, 64)),
    ("n2_t33_d16_h2_causal", (2, 33, 33, 16, 2, 0, 1, 65)),
]

PAD_MASKS = {5: np.array([[1, 1, 1, 1, 0], [1, 1, 1, 1, 1], [1, 1, 0, 0, 0]], np.float32)}


def attention_inputs(spec):
    N, Tq, Tk, D, heads, padded, causal, seed = spec
    q, k, v, g = synth.uniform_operands(seed, [(N, Tq, D), (N, Tk, D), (N, Tk, D), (N, Tq, D)], -2.0, 2.0)
    mask = np.ascontiguousarray(PAD_MASKS[Tk][:N]) if padded else None
    return (np.ascontiguousarray(q), np.ascontiguousarray(k), np.ascontiguousarray(v), heads, mask, causal,
            np.ascontiguousarray(g))


# name, (N, C, H, W, kernel, stride, seed, specials): specials quantises the input to quarters (ties), fills one
# window with -inf (nothing beats the start value: offset 0 keeps the gradient), one with NaN and plants a NaN
# among ordinary values
POOL_CASES = [
    ("k2s2_2x3x8x8", (2, 3, 8, 8, 2, 2, 61, 0)),
    ("k3s2_overlap_1x2x9x7_specials", (1, 2, 9, 7, 3, 2, 62, 1)),
    ("k3s1_overlap_1x1x6x6_specials", (1, 1, 6, 6, 3, 1, 63, 1)),
    ("k2s1_ties_1x2x5x5_specials", (1, 2, 5, 5, 2, 1, 64, 1)),
    ("k2s2_odd_2x2x7x9", (2, 2, 7, 9, 2, 2, 65, 0)),
    ("k2s2_specials_2x2x6x6", (2, 2, 6, 6, 2, 2, 66, 1)),
]


def pool_inputs(spec):
    N, C, H, W, k, s, seed, specials = spec
    ho, wo = (H - k) // s + 1, (W - k) // s + 1
    x, g = synth.uniform_operands(seed, [(N, C, H, W), (N, C, ho, wo)])
    x = np.array(x, copy=True)
    if specials:
        x = (np.round(x * 4) / 4).astype(np.float32)
        x[0, 0, H - k:H, W - k:W] = -np.inf                      # the last window: nothing above -inf
        x[-1, -1, 0:k, 0:k] = np.nan                             # the first window of the last plane: all NaN
        x[0, -1, H // 2, W // 2] = np.nan                        # a NaN among ordinary values
    return np.ascontiguousarray(x), np.ascontiguousarray(g), k, s


# nn::batchnorm in training mode on {N, C, S...}: (N, C, spatial shape, relu, seed). Inputs: x from U[-3, 5], weight
# from U[0.5, 1.5], bias from U[-1, 1], the upstream gradient from U[-1, 1].
BATCHNORM_CASES = [
    ("bn2d_4x3x5x5", (4, 3, (5, 5), 0, 71)),
    ("bn2d_relu_4x3x5x5", (4, 3, (5, 5), 1, 72)),
    ("bn1d_16x4", (16, 4, (), 0, 73)),
    ("bn2d_relu_tail_3x2x3x7", (3, 2, (3, 7), 1, 74)),
    ("bn2d_one_element_per_channel_1x3x1x1", (1, 3, (1, 1), 0, 75)),
]


def batchnorm_inputs(spec):
    N, C, sp, relu, seed = spec
    shape = (N, C) + tuple(sp)
    x, w, b, g = synth.uniform_operands(seed, [shape, (C,), (C,), shape])
    x = (x * 4 + 1).astype(np.float32)
    w = (w * 0.5 + 1).astype(np.float32)
    return np.ascontiguousarray(x), np.ascontiguousarray(w), np.ascontiguousarray(b), np.ascontiguousarray(g), relu


# nn::layernorm over the last axis: (shape, seed). x from U[-2, 3], gamma U[0.5, 1.5], beta U[-1, 1].
LAYERNORM_CASES = [
    ("ln_2x7", ((2, 7), 76)),
    ("ln_2x3x5", ((2, 3, 5), 77)),
    ("ln_16x64", ((16, 64), 78)),
    ("ln_3x1", ((3, 1), 79)),
]


def layernorm_inputs(spec):
    shape, seed = spec
    D = shape[-1]
    x, gm, bt, g = synth.uniform_operands(seed, [shape, (D,), (D,), shape])
    x = (x * 2.5 + 0.5).astype(np.float32)
    gm = (gm * 0.5 + 1).astype(np.float32)
    return np.ascontiguousarray(x), np.ascontiguousarray(gm), np.ascontiguousarray(bt), np.ascontiguousarray(g)

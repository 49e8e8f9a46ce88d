"""ctypes access to the CPU checker (oracle/lib/liboracle.so) and to nn-cpp itself (oracle/_ref/libnnref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
never by the product package. All arrays are numpy float32 (row-major); results are returned as new
arrays so a caller never aliases the checker's buffers.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "lib", "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libnnref.so")
REF_HIP_SO = os.path.join(HERE, "_ref", "libnnref_hip.so")  # nn-cpp with its GEMM replaced by the GPU drop-in

_f = C.POINTER(C.c_float)
_d = C.POINTER(C.c_double)
_u8 = C.POINTER(C.c_ubyte)
_sz = C.c_size_t
_szp = C.POINTER(C.c_size_t)


def _fp(a):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_f)


def _dp(a):
    if a is None:
        return None
    assert a.dtype == np.float64 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_d)


def _bp(a):
    if a is None:
        return None
    assert a.dtype == np.uint8 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_u8)


class Oracle:
    """The C restatement (bit-exact emulation of nn-cpp's NN_NATIVE arithmetic) and fp64 closed forms."""

    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle` (or __graft_entry__.build())")
        L = self.lib = C.CDLL(path)
        gemm = [C.c_int, C.c_int, _sz, _sz, _sz, _f, _sz, _f, _sz, _f, _sz, C.c_int]
        for name in ("oracle_sgemm", "oracle_sgemm_naive"):
            getattr(L, name).argtypes = gemm
            getattr(L, name).restype = None
        L.oracle_sgemm_at.argtypes = [C.c_int, C.c_int, _sz, _sz, _sz, _f, _sz, _f, _sz, C.c_int, _szp, _szp, _f,
                                      _sz, _f]
        L.oracle_depth_cut.argtypes = [_sz, _sz, _sz]
        L.oracle_depth_cut.restype = C.c_int
        L.oracle_piece_depth.argtypes = [_sz, _sz, _sz]
        L.oracle_piece_depth.restype = _sz
        L.oracle_set_numerics.argtypes = [C.c_int]
        L.oracle_sgemm_f64.argtypes = [C.c_int, C.c_int, _sz, _sz, _sz, _f, _sz, _f, _sz, _f, _sz, C.c_int, _d, _d]
        L.oracle_sum_axis0.argtypes = [_f, _sz, _sz, _f]
        L.oracle_lane_sum.argtypes = [_f, _sz]
        L.oracle_lane_sum.restype = C.c_float
        L.oracle_linear_forward.argtypes = [_f, _sz, _sz, _f, _sz, _f, _f]
        L.oracle_linear_backward.argtypes = [_f, _f, _f, _sz, _sz, _sz, _szp, C.c_int, _f, C.c_int, _f, C.c_int,
                                             _f, C.c_int]
        L.oracle_relu.argtypes = [_f, _f, _sz]
        L.oracle_im2col_sample.argtypes = [_f, _f, _sz, _sz, _sz, _sz, _sz, _sz, _sz]
        L.oracle_col2im_sample_add.argtypes = [_f, _f, _sz, _sz, _sz, _sz, _sz, _sz, _sz]
        L.oracle_conv2d_forward.argtypes = [_f, _sz, _sz, _sz, _sz, _f, _sz, _sz, _sz, _f, _sz, _sz, C.c_int, _f, _u8]
        L.oracle_conv2d_backward.argtypes = [_f, _f, _f, _u8, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _f,
                                             C.c_int, _f, _f]
        L.oracle_conv2d_f64.argtypes = [_f, _sz, _sz, _sz, _sz, _f, _sz, _sz, _sz, _f, _sz, _sz, _d, _d]
        L.oracle_masked_softmax_row.argtypes = [_f, _f, _sz, _sz, _f, C.c_int, C.c_float]
        L.oracle_attention_forward.argtypes = [_f, _f, _f, _sz, _sz, _sz, _sz, _sz, _f, C.c_int, _f, _f]
        L.oracle_attention_backward.argtypes = [_f, _f, _f, _f, _f, _sz, _sz, _sz, _sz, _sz, _f, C.c_int,
                                                _f, C.c_int, _f, C.c_int, _f, C.c_int]
        L.oracle_scaled_masked_softmax.argtypes = [_f, _sz, _sz, _sz, _sz, C.c_float, _f, C.c_int, _f]
        L.oracle_scaled_masked_softmax_backward.argtypes = [_f, _f, _sz, _sz, _sz, _sz, C.c_float, _f, C.c_int, _f,
                                                             C.c_int]
        L.oracle_attention_f64.argtypes = [_f, _f, _f, _sz, _sz, _sz, _sz, _sz, _f, C.c_int, _d, _d]
        L.oracle_mt19937_uniform.argtypes = [C.c_uint, C.c_float, C.c_float, _f, _sz]
        _u32 = C.POINTER(C.c_uint32)
        L.oracle_batchnorm_forward.argtypes = [_f, _sz, _sz, _sz, _f, _f, C.c_float, C.c_int, _f, _u8, _f, _f, _f]
        L.oracle_batchnorm_backward.argtypes = [_f, _f, _u8, _f, _f, _f, _sz, _sz, _sz, _f, C.c_int, _f, C.c_int, _f,
                                                C.c_int]
        L.oracle_layernorm_forward.argtypes = [_f, _sz, _sz, _f, _f, C.c_float, _f, _f, _f]
        L.oracle_layernorm_backward.argtypes = [_f, _f, _f, _f, _f, _sz, _sz, _f, C.c_int, _f, C.c_int, _f, C.c_int]
        L.oracle_batchnorm_f64.argtypes = [_f, _sz, _sz, _sz, C.c_double, _d]
        L.oracle_layernorm_f64.argtypes = [_f, _sz, _sz, C.c_double, _d]
        L.oracle_tanh_one.argtypes = [C.c_float]
        L.oracle_tanh_one.restype = C.c_float
        L.oracle_gelu_forward.argtypes = [_f, _sz, _f, _f]
        L.oracle_gelu_backward.argtypes = [_f, _f, _f, _sz, _f, C.c_int]
        L.oracle_embedding_backward.argtypes = [_f, C.POINTER(C.c_int32), _sz, _sz, _sz, _f, C.c_int]
        L.oracle_maxpool2d_forward.argtypes = [_f, _sz, _sz, _sz, _sz, _sz, _f, _u32]
        L.oracle_maxpool2d_backward.argtypes = [_f, _u32, _sz, _sz, _sz, _sz, _sz, _f, C.c_int]

    # -- GEMM --
    def sgemm(self, ta, tb, m, n, k, a, lda, b, ldb, c, ldc, acc, naive=False):
        """Returns a copy of c updated by nn::kernels::sgemm's arithmetic (or the naive fp32 triple loop)."""
        out = np.array(c, dtype=np.float32, copy=True)
        fn = self.lib.oracle_sgemm_naive if naive else self.lib.oracle_sgemm
        fn(int(ta), int(tb), m, n, k, _fp(a), lda, _fp(b), ldb, _fp(out), ldc, int(acc))
        return out

    def sgemm_at(self, ta, tb, m, n, k, a, lda, b, ldb, acc, rows, cols, c_old=None):
        """sgemm's value at elements (rows[t], cols[t]); c_old holds those elements before the call."""
        rows = np.ascontiguousarray(rows, np.uint64)
        cols = np.ascontiguousarray(cols, np.uint64)
        cnt = rows.size
        cold = np.ascontiguousarray(c_old if c_old is not None else np.zeros(cnt), np.float32)
        out = np.empty(cnt, np.float32)
        self.lib.oracle_sgemm_at(int(ta), int(tb), m, n, k, _fp(a), lda, _fp(b), ldb, int(acc),
                                 rows.ctypes.data_as(_szp), cols.ctypes.data_as(_szp), _fp(cold), cnt, _fp(out))
        return out

    def set_numerics(self, mode):
        """0: nn-cpp's depth-cut rule; 1: the split-depth rule of the library's NNH_NUMERICS_SPLIT_DEPTH."""
        self.lib.oracle_set_numerics(int(mode))

    def depth_cut(self, m, n, k):
        return bool(self.lib.oracle_depth_cut(m, n, k))

    def piece_depth(self, m, n, k):
        """Depth of one piece of a cut product (0: not cut)."""
        return int(self.lib.oracle_piece_depth(m, n, k))

    def sgemm_f64(self, ta, tb, m, n, k, a, lda, b, ldb, c, ldc, acc):
        """fp64 op(A) op(B) (+ C) as a dense m x n array, with the magnitude sum |a||b| (+|c|)."""
        out = np.zeros((m, n), np.float64)
        mag = np.zeros((m, n), np.float64)
        cin = c if c is not None else np.zeros(1, np.float32)
        self.lib.oracle_sgemm_f64(int(ta), int(tb), m, n, k, _fp(a), lda, _fp(b), ldb, _fp(cin), ldc, int(acc),
                                  _dp(out), _dp(mag))
        return out, mag

    # -- reductions --
    def sum_axis0(self, src):
        src = np.ascontiguousarray(src, np.float32)
        rows, inner = src.shape[0], int(np.prod(src.shape[1:], dtype=np.int64))
        out = np.empty(src.shape[1:], np.float32)
        self.lib.oracle_sum_axis0(_fp(src), rows, inner, _fp(out))
        return out

    def lane_sum(self, p):
        p = np.ascontiguousarray(p, np.float32)
        return np.float32(self.lib.oracle_lane_sum(_fp(p), p.size))

    # -- linear --
    def linear_forward(self, x, w, bias):
        K = x.shape[-1]
        M = x.size // K
        n = w.shape[0]
        y = np.empty(x.shape[:-1] + (n,), np.float32)
        self.lib.oracle_linear_forward(_fp(x), M, K, _fp(w), n, _fp(bias), _fp(y))
        return y

    def linear_backward(self, g, x, w, dx=None, dx_first=True, dw=None, dw_first=True, db=None, db_first=True,
                        want=(True, True, True)):
        K = x.shape[-1]
        M = x.size // K
        n = w.shape[0]
        lead = (C.c_size_t * max(1, x.ndim - 1))(*x.shape[:-1])
        dx = (np.array(dx, np.float32) if dx is not None else np.zeros(x.shape, np.float32)) if want[0] else None
        dw = (np.array(dw, np.float32) if dw is not None else np.zeros(w.shape, np.float32)) if want[1] else None
        db = (np.array(db, np.float32) if db is not None else np.zeros((n,), np.float32)) if want[2] else None
        self.lib.oracle_linear_backward(_fp(g), _fp(x), _fp(w), M, K, n, lead, x.ndim - 1, _fp(dx), int(dx_first),
                                        _fp(dw), int(dw_first), _fp(db), int(db_first))
        return dx, dw, db

    def relu(self, x):
        y = np.empty_like(x)
        self.lib.oracle_relu(_fp(x), _fp(y), x.size)
        return y

    # -- conv --
    @staticmethod
    def conv_out(H, W, kh, kw, stride, pad):
        return (H + 2 * pad - kh) // stride + 1, (W + 2 * pad - kw) // stride + 1

    def im2col(self, x, kh, kw, stride, pad):
        N, Cin, H, W = x.shape
        ho, wo = self.conv_out(H, W, kh, kw, stride, pad)
        col = np.empty((N, Cin * kh * kw, ho * wo), np.float32)
        for n in range(N):
            xs = np.ascontiguousarray(x[n])
            cs = np.empty((Cin * kh * kw, ho * wo), np.float32)
            self.lib.oracle_im2col_sample(_fp(xs), _fp(cs), Cin, H, W, kh, kw, stride, pad)
            col[n] = cs
        return col

    def col2im_add(self, col, dx, kh, kw, stride, pad):
        dx = np.array(dx, np.float32, copy=True)
        N, Cin, H, W = dx.shape
        for n in range(N):
            cs = np.ascontiguousarray(col[n])
            xs = np.ascontiguousarray(dx[n])
            self.lib.oracle_col2im_sample_add(_fp(cs), _fp(xs), Cin, H, W, kh, kw, stride, pad)
            dx[n] = xs
        return dx

    def conv2d_forward(self, x, w, bias, stride, pad, fuse_relu):
        N, Cin, H, W = x.shape
        Cout, _, kh, kw = w.shape
        ho, wo = self.conv_out(H, W, kh, kw, stride, pad)
        y = np.empty((N, Cout, ho, wo), np.float32)
        alive = np.zeros((N, Cout, ho, wo), np.uint8)
        self.lib.oracle_conv2d_forward(_fp(x), N, Cin, H, W, _fp(w), Cout, kh, kw, _fp(bias), stride, pad,
                                       int(fuse_relu), _fp(y), _bp(alive))
        return y, alive

    def conv2d_backward(self, g, x, w, alive, stride, pad, dx=None, dx_first=True):
        N, Cin, H, W = x.shape
        Cout, _, kh, kw = w.shape
        dx = np.array(dx, np.float32) if dx is not None else np.zeros(x.shape, np.float32)
        dw = np.zeros(w.shape, np.float32)
        db = np.zeros((Cout,), np.float32)
        self.lib.oracle_conv2d_backward(_fp(g), _fp(x), _fp(w), _bp(alive), N, Cin, H, W, Cout, kh, kw, stride, pad,
                                        _fp(dx), int(dx_first), _fp(dw), _fp(db))
        return dx, dw, db

    def conv2d_f64(self, x, w, bias, stride, pad):
        N, Cin, H, W = x.shape
        Cout, _, kh, kw = w.shape
        ho, wo = self.conv_out(H, W, kh, kw, stride, pad)
        y = np.empty((N, Cout, ho, wo), np.float64)
        mag = np.empty_like(y)
        self.lib.oracle_conv2d_f64(_fp(x), N, Cin, H, W, _fp(w), Cout, kh, kw, _fp(bias), stride, pad, _dp(y), _dp(mag))
        return y, mag

    # -- attention --
    def attention_forward(self, q, k, v, heads, pad=None, causal=False):
        N, Tq, D = q.shape
        Tk = k.shape[1]
        out = np.empty((N, Tq, D), np.float32)
        probs = np.empty((N, heads, Tq, Tk), np.float32)
        self.lib.oracle_attention_forward(_fp(q), _fp(k), _fp(v), N, Tq, Tk, D, heads, _fp(pad), int(causal),
                                          _fp(out), _fp(probs))
        return out, probs

    def attention_backward(self, g, q, k, v, probs, heads, pad=None, causal=False):
        N, Tq, D = q.shape
        Tk = k.shape[1]
        dq, dk, dv = (np.zeros(q.shape, np.float32), np.zeros(k.shape, np.float32), np.zeros(v.shape, np.float32))
        self.lib.oracle_attention_backward(_fp(g), _fp(q), _fp(k), _fp(v), _fp(probs), N, Tq, Tk, D, heads, _fp(pad),
                                           int(causal), _fp(dq), 1, _fp(dk), 1, _fp(dv), 1)
        return dq, dk, dv

    def scaled_masked_softmax(self, x, scale, pad=None, causal=False):
        N, H, Tq, Tk = x.shape
        y = np.empty_like(x)
        self.lib.oracle_scaled_masked_softmax(_fp(x), N, H, Tq, Tk, scale, _fp(pad), int(causal), _fp(y))
        return y

    def scaled_masked_softmax_backward(self, y, g, scale, pad=None, causal=False, dx=None, first=True):
        N, H, Tq, Tk = y.shape
        out = np.array(dx, np.float32, copy=True) if dx is not None else np.zeros_like(y)
        self.lib.oracle_scaled_masked_softmax_backward(_fp(np.ascontiguousarray(y, np.float32)),
                                                       _fp(np.ascontiguousarray(g, np.float32)), N, H, Tq, Tk, scale,
                                                       _fp(pad), int(causal), _fp(out), int(first))
        return out

    def attention_f64(self, q, k, v, heads, pad=None, causal=False):
        N, Tq, D = q.shape
        Tk = k.shape[1]
        out = np.empty((N, Tq, D), np.float64)
        probs = np.empty((N, heads, Tq, Tk), np.float64)
        self.lib.oracle_attention_f64(_fp(q), _fp(k), _fp(v), N, Tq, Tk, D, heads, _fp(pad), int(causal),
                                      _dp(out), _dp(probs))
        return out, probs

    # -- max pooling --
    def maxpool2d_forward(self, x, k, s):
        """(y, argmax) of nn::maxpool2d on x {N, C, H, W}."""
        x = np.ascontiguousarray(x, np.float32)
        N, Cc, H, W = x.shape
        ho, wo = (H - k) // s + 1, (W - k) // s + 1
        y = np.empty((N, Cc, ho, wo), np.float32)
        arg = np.empty((N, Cc, ho, wo), np.uint32)
        self.lib.oracle_maxpool2d_forward(_fp(x), N * Cc, H, W, k, s, _fp(y), arg.ctypes.data_as(C.POINTER(C.c_uint32)))
        return y, arg

    def maxpool2d_backward(self, g, argmax, x_shape, k, s, dx=None, first=True):
        N, Cc, H, W = x_shape
        out = np.array(dx, np.float32, copy=True) if dx is not None else np.empty(x_shape, np.float32)
        g = np.ascontiguousarray(g, np.float32)
        argmax = np.ascontiguousarray(argmax, np.uint32)
        self.lib.oracle_maxpool2d_backward(_fp(g), argmax.ctypes.data_as(C.POINTER(C.c_uint32)), N * Cc, H, W, k, s,
                                           _fp(out), int(first))
        return out

    # -- normalisation --
    @staticmethod
    def _nsc(x):
        """(N, C, S) of a {N, C, ...} array."""
        S = 1
        for d in x.shape[2:]:
            S *= d
        return x.shape[0], x.shape[1], S

    def batchnorm_forward(self, x, w, b, eps, relu=False):
        """(y, alive or None, mean, var, inv_std) of nn::batchnorm in training mode on x {N, C, ...}."""
        x = np.ascontiguousarray(x, np.float32)
        N, Cc, S = self._nsc(x)
        y = np.empty_like(x)
        alive = np.empty(x.shape, np.uint8) if relu else None
        mean, var, inv = (np.empty(Cc, np.float32) for _ in range(3))
        self.lib.oracle_batchnorm_forward(_fp(x), N, Cc, S, _fp(np.ascontiguousarray(w, np.float32)),
                                          _fp(np.ascontiguousarray(b, np.float32)), float(eps), int(relu), _fp(y),
                                          _bp(alive), _fp(mean), _fp(var), _fp(inv))
        return y, alive, mean, var, inv

    def batchnorm_backward(self, g, x, alive, w, mean, inv_std, dx=None, dx_first=True, dw=None, dw_first=True,
                           db=None, db_first=True, want=(True, True, True)):
        """(dx, dw, db) of the backward rule; an output is None where `want` says so. Existing dx/dw/db arrays are
        the buffers added to when the matching *_first is false."""
        x = np.ascontiguousarray(x, np.float32)
        N, Cc, S = self._nsc(x)
        outs = []
        for buf, shape, wanted in ((dx, x.shape, want[0]), (dw, (Cc,), want[1]), (db, (Cc,), want[2])):
            outs.append((np.array(buf, np.float32, copy=True) if buf is not None else np.zeros(shape, np.float32))
                        if wanted else None)
        self.lib.oracle_batchnorm_backward(_fp(np.ascontiguousarray(g, np.float32)), _fp(x), _bp(alive),
                                           _fp(np.ascontiguousarray(w, np.float32)), _fp(mean), _fp(inv_std), N, Cc, S,
                                           _fp(outs[0]), int(dx_first), _fp(outs[1]), int(dw_first), _fp(outs[2]),
                                           int(db_first))
        return tuple(outs)

    def layernorm_forward(self, x, gamma, beta, eps):
        """(y, mean, inv_std) of nn::layernorm over the last axis."""
        x = np.ascontiguousarray(x, np.float32)
        D = x.shape[-1]
        R = x.size // D
        y = np.empty_like(x)
        mean, inv = np.empty(R, np.float32), np.empty(R, np.float32)
        self.lib.oracle_layernorm_forward(_fp(x), R, D, _fp(np.ascontiguousarray(gamma, np.float32)),
                                          _fp(np.ascontiguousarray(beta, np.float32)), float(eps), _fp(y), _fp(mean),
                                          _fp(inv))
        return y, mean, inv

    def layernorm_backward(self, g, x, gamma, mean, inv_std, dx=None, dx_first=True, dgamma=None, dgamma_first=True,
                           dbeta=None, dbeta_first=True, want=(True, True, True)):
        x = np.ascontiguousarray(x, np.float32)
        D = x.shape[-1]
        R = x.size // D
        outs = []
        for buf, shape, wanted in ((dx, x.shape, want[0]), (dgamma, (D,), want[1]), (dbeta, (D,), want[2])):
            outs.append((np.array(buf, np.float32, copy=True) if buf is not None else np.zeros(shape, np.float32))
                        if wanted else None)
        self.lib.oracle_layernorm_backward(_fp(np.ascontiguousarray(g, np.float32)), _fp(x),
                                           _fp(np.ascontiguousarray(gamma, np.float32)), _fp(mean), _fp(inv_std), R, D,
                                           _fp(outs[0]), int(dx_first), _fp(outs[1]), int(dgamma_first), _fp(outs[2]),
                                           int(dbeta_first))
        return tuple(outs)

    def gelu_forward(self, x):
        """(y, th) of nn::gelu, th the tanh it keeps for the backward pass."""
        x = np.ascontiguousarray(x, np.float32)
        y, th = np.empty_like(x), np.empty_like(x)
        self.lib.oracle_gelu_forward(_fp(x), x.size, _fp(y), _fp(th))
        return y, th

    def gelu_backward(self, x, th, g, dx=None, first=True):
        x = np.ascontiguousarray(x, np.float32)
        out = np.array(dx, np.float32, copy=True) if dx is not None else np.empty_like(x)
        self.lib.oracle_gelu_backward(_fp(x), _fp(np.ascontiguousarray(th, np.float32)),
                                      _fp(np.ascontiguousarray(g, np.float32)), x.size, _fp(out), int(first))
        return out

    def embedding_backward(self, g, rows, V, D, dw=None, first=True):
        g = np.ascontiguousarray(g, np.float32)
        rows = np.ascontiguousarray(rows, np.int32)
        out = np.array(dw, np.float32, copy=True) if dw is not None else np.empty((V, D), np.float32)
        self.lib.oracle_embedding_backward(_fp(g), rows.ctypes.data_as(C.POINTER(C.c_int32)), rows.size, V, D,
                                           _fp(out), int(first))
        return out

    def batchnorm_f64(self, x, eps):
        x = np.ascontiguousarray(x, np.float32)
        N, Cc, S = self._nsc(x)
        out = np.empty(x.shape, np.float64)
        self.lib.oracle_batchnorm_f64(_fp(x), N, Cc, S, float(eps), _dp(out))
        return out

    def layernorm_f64(self, x, eps):
        x = np.ascontiguousarray(x, np.float32)
        D = x.shape[-1]
        out = np.empty(x.shape, np.float64)
        self.lib.oracle_layernorm_f64(_fp(x), x.size // D, D, float(eps), _dp(out))
        return out

    def mt19937_uniform(self, seed, lo, hi, count):
        out = np.empty(count, np.float32)
        self.lib.oracle_mt19937_uniform(seed, lo, hi, _fp(out), count)
        return out


class Reference:
    """nn-cpp itself (its unmodified sources compiled by oracle/Makefile), through oracle/ref_shim.cpp."""

    def __init__(self, path=REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle ref` where /root/reference exists")
        L = self.lib = C.CDLL(path)
        L.nnref_set_threads.argtypes = [_sz]
        L.nnref_num_threads.restype = _sz
        L.nnref_uses_avx2.restype = C.c_int
        L.nnref_sgemm.argtypes = [C.c_int, C.c_int, _sz, _sz, _sz, _f, _sz, _f, _sz, _f, _sz, C.c_int]
        L.nnref_sgemm_portable.argtypes = L.nnref_sgemm.argtypes
        L.nnref_sgemm_unpacked.argtypes = L.nnref_sgemm.argtypes
        L.nnref_matmul.argtypes = [_f, _szp, C.c_int, _f, _szp, C.c_int, C.c_int, C.c_int, _f, _sz, _szp,
                                   C.POINTER(C.c_int)]
        L.nnref_linear_forward.argtypes = [_f, _szp, C.c_int, _f, _sz, _f, _f]
        L.nnref_linear_backward.argtypes = [_f, _szp, C.c_int, _f, _sz, _f, _f, _f, _f, _f]
        L.nnref_conv2d_forward.argtypes = [_f, _sz, _sz, _sz, _sz, _f, _sz, _sz, _sz, _f, C.c_int, C.c_int, C.c_int, _f]
        L.nnref_conv2d_backward.argtypes = [_f, _sz, _sz, _sz, _sz, _f, _sz, _sz, _sz, _f, C.c_int, C.c_int, C.c_int,
                                            _f, _f, _f, _f]
        L.nnref_attention_forward.argtypes = [_f, _f, _f, _sz, _sz, _sz, _sz, _sz, _f, C.c_int, _f]
        L.nnref_attention_backward.argtypes = [_f, _f, _f, _sz, _sz, _sz, _sz, _sz, _f, C.c_int, _f, _f, _f, _f]
        L.nnref_scaled_masked_softmax.argtypes = [_f, _sz, _sz, _sz, _sz, C.c_float, _f, C.c_int, _f]
        L.nnref_module_run.argtypes = [C.c_int, C.c_uint, _f, _szp, C.c_int, _f, _f, _sz, _f, _sz, _szp, _szp]
        L.nnref_maxpool2d.argtypes = [_f, _sz, _sz, _sz, _sz, _sz, _sz, _f, _f, _f]
        L.nnref_time_maxpool2d.argtypes = [_f, _sz, _sz, _sz, _sz, _sz, _sz, _f, C.c_int, C.c_int, C.c_double, _d,
                                           C.POINTER(C.c_int), _d, _f, _f]
        L.nnref_matmul_backward.argtypes = [_f, _szp, C.c_int, _f, _szp, C.c_int, C.c_int, _f, C.c_int, _f, _f]
        L.nnref_batchnorm.argtypes = [_f, _sz, _sz, _sz, _f, _f, C.c_float, C.c_int, _f, _f, _f, _f, C.c_int, _f, _f,
                                      _f]
        L.nnref_layernorm.argtypes = [_f, _sz, _sz, _f, _f, C.c_float, _f, _f, C.c_int, _f, _f, _f]
        L.nnref_gelu.argtypes = [_f, _sz, _f, _f, C.c_int, _f]
        L.nnref_embedding.argtypes = [_f, _sz, _sz, _f, _sz, _f, _f, C.c_int, _f]
        L.nnref_transformer_tiny_layout.argtypes = [_szp, _sz, _szp]
        L.nnref_time_batchnorm.argtypes = [_f, _sz, _sz, _sz, _f, _f, C.c_float, C.c_int, _f, C.c_int, C.c_int,
                                           C.c_double, _d, C.POINTER(C.c_int), _d, _f, _f]
        L.nnref_time_layernorm.argtypes = [_f, _sz, _sz, _f, _f, C.c_float, _f, C.c_int, C.c_int, C.c_double, _d,
                                           C.POINTER(C.c_int), _d, _f, _f]
        _fpp = C.POINTER(_f)
        timing = [C.c_int, C.c_int, C.c_double, _d]
        L.nnref_time_matmul.argtypes = [_f, _szp, C.c_int, _f, _szp, C.c_int, C.c_int, C.c_int] + timing + [_f]
        L.nnref_time_linear_relu_chain.argtypes = [_f, _sz, _szp, C.c_int, _fpp, _fpp] + timing + [_fpp]
        L.nnref_time_linear_backward_layers.argtypes = [_fpp, _sz, _szp, C.c_int, _fpp, _fpp, _fpp] + timing + \
            [_fpp, _fpp, _fpp]
        L.nnref_time_conv2d.argtypes = [_f, _sz, _sz, _sz, _sz, _f, _sz, _sz, _sz, _f, C.c_int, C.c_int, C.c_int, _f] + \
            timing[:3] + [_d, C.POINTER(C.c_int), _d, _f, _f, _f, _f]
        L.nnref_time_attention.argtypes = [_f, _f, _f, _sz, _sz, _sz, _sz, C.c_int, _f] + timing[:3] + \
            [_d, C.POINTER(C.c_int), _d, _f, _f, _f, _f]

    def set_threads(self, n):
        self.lib.nnref_set_threads(n)

    def num_threads(self):
        return int(self.lib.nnref_num_threads())

    def uses_avx2(self):
        return bool(self.lib.nnref_uses_avx2())

    def sgemm(self, ta, tb, m, n, k, a, lda, b, ldb, c, ldc, acc):
        out = np.array(c, dtype=np.float32, copy=True)
        self.lib.nnref_sgemm(int(ta), int(tb), m, n, k, _fp(a), lda, _fp(b), ldb, _fp(out), ldc, int(acc))
        return out

    def sgemm_variant(self, name, ta, tb, m, n, k, a, lda, b, ldb, c, ldc, acc):
        """nn::kernels::sgemm_portable ("portable") or sgemm_unpacked ("unpacked") on a copy of c."""
        out = np.array(c, dtype=np.float32, copy=True)
        getattr(self.lib, f"nnref_sgemm_{name}")(int(ta), int(tb), m, n, k, _fp(a), lda, _fp(b), ldb, _fp(out), ldc,
                                                  int(acc))
        return out

    def sgemm_inplace(self, ta, tb, m, n, k, a, lda, b, ldb, c, ldc, acc):
        self.lib.nnref_sgemm(int(ta), int(tb), m, n, k, _fp(a), lda, _fp(b), ldb, _fp(c), ldc, int(acc))

    def matmul(self, a, b, ta=False, tb=False):
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        ash = (C.c_size_t * a.ndim)(*a.shape)
        bsh = (C.c_size_t * b.ndim)(*b.shape)
        cap = max(1, (a.size + 1) * (b.size + 1))
        cap = min(cap, 1 << 26)
        out = np.empty(cap, np.float32)
        osh = (C.c_size_t * 8)()
        ond = C.c_int(0)
        rc = self.lib.nnref_matmul(_fp(a), ash, a.ndim, _fp(b), bsh, b.ndim, int(ta), int(tb), _fp(out), cap, osh,
                                   C.byref(ond))
        if rc != 0:
            return rc, None
        shape = tuple(osh[i] for i in range(ond.value))
        return 0, out[: int(np.prod(shape, dtype=np.int64))].reshape(shape).copy()

    def linear_forward(self, x, w, bias):
        xs = (C.c_size_t * x.ndim)(*x.shape)
        y = np.empty(x.shape[:-1] + (w.shape[0],), np.float32)
        rc = self.lib.nnref_linear_forward(_fp(x), xs, x.ndim, _fp(w), w.shape[0], _fp(bias), _fp(y))
        assert rc == 0, rc
        return y

    def linear_backward(self, x, w, bias, g):
        xs = (C.c_size_t * x.ndim)(*x.shape)
        dx, dw, db = np.empty_like(x), np.empty_like(w), np.empty_like(bias)
        rc = self.lib.nnref_linear_backward(_fp(x), xs, x.ndim, _fp(w), w.shape[0], _fp(bias), _fp(g), _fp(dx),
                                            _fp(dw), _fp(db))
        assert rc == 0, rc
        return dx, dw, db

    def conv2d_forward(self, x, w, bias, stride, pad, fuse_relu):
        N, Cin, H, W = x.shape
        Cout, _, kh, kw = w.shape
        ho, wo = Oracle.conv_out(H, W, kh, kw, stride, pad)
        y = np.empty((N, Cout, ho, wo), np.float32)
        rc = self.lib.nnref_conv2d_forward(_fp(x), N, Cin, H, W, _fp(w), Cout, kh, kw, _fp(bias), stride, pad,
                                           int(fuse_relu), _fp(y))
        assert rc == 0, rc
        return y

    def conv2d_backward(self, x, w, bias, stride, pad, fuse_relu, g):
        N, Cin, H, W = x.shape
        Cout, _, kh, kw = w.shape
        dx, dw, db = np.empty_like(x), np.empty_like(w), np.empty_like(bias)
        rc = self.lib.nnref_conv2d_backward(_fp(x), N, Cin, H, W, _fp(w), Cout, kh, kw, _fp(bias), stride, pad,
                                            int(fuse_relu), _fp(g), _fp(dx), _fp(dw), _fp(db))
        assert rc == 0, rc
        return dx, dw, db

    def attention_forward(self, q, k, v, heads, pad=None, causal=False):
        N, Tq, D = q.shape
        Tk = k.shape[1]
        out = np.empty((N, Tq, D), np.float32)
        rc = self.lib.nnref_attention_forward(_fp(q), _fp(k), _fp(v), N, Tq, Tk, D, heads, _fp(pad), int(causal),
                                              _fp(out))
        assert rc == 0, rc
        return out

    def attention_backward(self, q, k, v, heads, g, pad=None, causal=False):
        N, Tq, D = q.shape
        Tk = k.shape[1]
        dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
        rc = self.lib.nnref_attention_backward(_fp(q), _fp(k), _fp(v), N, Tq, Tk, D, heads, _fp(pad), int(causal),
                                               _fp(g), _fp(dq), _fp(dk), _fp(dv))
        assert rc == 0, rc
        return dq, dk, dv

    def scaled_masked_softmax(self, x, scale, pad=None, causal=False):
        N, H, Tq, Tk = x.shape
        y = np.empty_like(x)
        rc = self.lib.nnref_scaled_masked_softmax(_fp(x), N, H, Tq, Tk, scale, _fp(pad), int(causal), _fp(y))
        assert rc == 0, rc
        return y


    def matmul_backward(self, a, b, bt, g, repeats=1):
        """(da, db) of nn::matmul (bt False) or nn::matmul_bt: the backward rule applied `repeats` times (fresh, then
        added)."""
        same = b is None
        b = a if same else b
        a, b, g = (np.ascontiguousarray(t, np.float32) for t in (a, b, g))
        da, db = np.empty_like(a), np.empty_like(b)
        rc = self.lib.nnref_matmul_backward(_fp(a), (C.c_size_t * a.ndim)(*a.shape), a.ndim, None if same else _fp(b),
                                            (C.c_size_t * b.ndim)(*b.shape), b.ndim, int(bt), _fp(g), repeats,
                                            _fp(da), _fp(db))
        assert rc == 0, rc
        return (da, None) if same else (da, db)

    def module_run(self, which, seed, x, g, out_cap=1 << 20, grads_cap=1 << 22):
        """nn-cpp module `which` (see nnref_module_run) built after manual_seed(seed): (output, all gradients)."""
        x, g = np.ascontiguousarray(x, np.float32), np.ascontiguousarray(g, np.float32)
        out, grads = np.empty(out_cap, np.float32), np.empty(grads_cap, np.float32)
        n_out, n_grads = C.c_size_t(0), C.c_size_t(0)
        rc = self.lib.nnref_module_run(which, seed, _fp(x), (C.c_size_t * x.ndim)(*x.shape), x.ndim, _fp(g), _fp(out),
                                       out_cap, _fp(grads), grads_cap, C.byref(n_out), C.byref(n_grads))
        assert rc == 0, rc
        return out[: n_out.value].copy(), grads[: n_grads.value].copy()

    def maxpool2d(self, x, k, s, g=None):
        """nn::maxpool2d's output and, given g, its input gradient (fresh)."""
        x = np.ascontiguousarray(x, np.float32)
        N, Cc, H, W = x.shape
        valid = k > 0 and s > 0 and k <= H and k <= W
        y = np.empty((N, Cc, (H - k) // s + 1, (W - k) // s + 1) if valid else (1,), np.float32)
        dx = np.empty_like(x)
        rc = self.lib.nnref_maxpool2d(_fp(x), N, Cc, H, W, k, s, _fp(y),
                                      _fp(np.ascontiguousarray(g, np.float32)) if g is not None else None, _fp(dx))
        if rc != 0:
            return rc, None, None
        return 0, y, (dx if g is not None else None)

    def batchnorm(self, x, w, b, eps, relu=False, g=None, repeats=1, want=(True, True, True)):
        """nn::batchnorm (training mode) on x {N, C, ...}: (rc, y, mean, var, (dx, dw, db) or None). With g, the node's
        backward rule runs `repeats` times (fresh gradients first, then added); `want` picks the inputs that require
        a gradient."""
        x = np.ascontiguousarray(x, np.float32)
        N, Cc, S = Oracle._nsc(x)
        y = np.empty_like(x)
        mean, var = np.empty(Cc, np.float32), np.empty(Cc, np.float32)
        grads = [np.empty(x.shape, np.float32) if want[0] else None, np.empty(Cc, np.float32) if want[1] else None,
                 np.empty(Cc, np.float32) if want[2] else None]
        rc = self.lib.nnref_batchnorm(_fp(x), N, Cc, S, _fp(np.ascontiguousarray(w, np.float32)),
                                      _fp(np.ascontiguousarray(b, np.float32)), float(eps), int(relu), _fp(y),
                                      _fp(mean), _fp(var), _fp(np.ascontiguousarray(g, np.float32)) if g is not None
                                      else None, int(repeats), *(_fp(t) for t in grads))
        if rc != 0:
            return rc, None, None, None, None
        return 0, y, mean, var, (tuple(grads) if g is not None else None)

    def layernorm(self, x, gamma, beta, eps, g=None, repeats=1, want=(True, True, True)):
        """nn::layernorm over the last axis: (rc, y, (dx, dgamma, dbeta) or None), as batchnorm()."""
        x = np.ascontiguousarray(x, np.float32)
        D = x.shape[-1]
        R = x.size // D
        y = np.empty_like(x)
        grads = [np.empty(x.shape, np.float32) if want[0] else None, np.empty(D, np.float32) if want[1] else None,
                 np.empty(D, np.float32) if want[2] else None]
        rc = self.lib.nnref_layernorm(_fp(x), R, D, _fp(np.ascontiguousarray(gamma, np.float32)),
                                      _fp(np.ascontiguousarray(beta, np.float32)), float(eps), _fp(y),
                                      _fp(np.ascontiguousarray(g, np.float32)) if g is not None else None,
                                      int(repeats), *(_fp(t) for t in grads))
        if rc != 0:
            return rc, None, None
        return 0, y, (tuple(grads) if g is not None else None)

    def gelu(self, x, g=None, repeats=1):
        """(rc, y, dx or None) of nn::gelu and its backward rule."""
        x = np.ascontiguousarray(x, np.float32)
        y, dx = np.empty_like(x), np.empty_like(x)
        rc = self.lib.nnref_gelu(_fp(x), x.size, _fp(y), _fp(np.ascontiguousarray(g, np.float32)) if g is not None
                                 else None, int(repeats), _fp(dx))
        return rc, y, (dx if g is not None else None)

    def embedding(self, w, ids, g=None, repeats=1):
        """(rc, y, dw or None) of nn::embedding; ids are floats, as nn-cpp takes them."""
        w = np.ascontiguousarray(w, np.float32)
        ids = np.ascontiguousarray(ids, np.float32)
        V, D = w.shape
        y = np.empty((ids.size, D), np.float32)
        dw = np.empty_like(w)
        rc = self.lib.nnref_embedding(_fp(w), V, D, _fp(ids), ids.size, _fp(y),
                                      _fp(np.ascontiguousarray(g, np.float32)) if g is not None else None, int(repeats),
                                      _fp(dw))
        return rc, (y if rc == 0 else None), (dw if g is not None and rc == 0 else None)

    def transformer_tiny_layout(self):
        """[(shape, starts_at_ones)] of nn-cpp's Transformer{64, 64, 4, 2, 64} parameters, in parameters() order."""
        buf = (C.c_size_t * 512)()
        n = C.c_size_t()
        assert self.lib.nnref_transformer_tiny_layout(buf, 512, C.byref(n)) == 0
        out, i = [], 0
        for _ in range(n.value):
            r = buf[i]
            out.append((tuple(buf[i + 1:i + 1 + r]), bool(buf[i + 1 + r])))
            i += r + 2
        return out

    # ---- timing (the CPU baseline): nn-cpp's own ops on buffers built once, apps/bench/runner.cpp's method ----
    # Each returns (times_ms, outputs): the timed runs after `warmup` untimed ones (at least one run, at most
    # max_runs, stopping once budget_s seconds of runs have passed) and the last run's outputs.

    @staticmethod
    def _times(buf, n):
        assert n >= 1, "nn-cpp raised an exception"
        return [float(buf[i]) for i in range(n)]

    def time_matmul(self, a, b, ta, tb, warmup, max_runs, budget_s):
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        m = a.shape[-1] if ta else a.shape[-2]
        n = b.shape[-2] if tb else b.shape[-1]
        out = np.empty(a.shape[:-2] + (m, n), np.float32)
        t = np.empty(max_runs, np.float64)
        ash, bsh = (C.c_size_t * a.ndim)(*a.shape), (C.c_size_t * b.ndim)(*b.shape)
        cnt = self.lib.nnref_time_matmul(_fp(a), ash, a.ndim, _fp(b), bsh, b.ndim, int(ta), int(tb), warmup, max_runs,
                                         budget_s, _dp(t), _fp(out))
        return self._times(t, cnt), out

    @staticmethod
    def _ptrs(arrs):
        return (_f * len(arrs))(*[_fp(x) for x in arrs])

    def time_linear_relu_chain(self, x, ws, bs, warmup, max_runs, budget_s):
        dims = [x.shape[1]] + [w.shape[0] for w in ws]
        M = x.shape[0]
        outs = [np.empty((M, d), np.float32) for d in dims[1:]]
        t = np.empty(max_runs, np.float64)
        cnt = self.lib.nnref_time_linear_relu_chain(_fp(x), M, (C.c_size_t * len(dims))(*dims), len(ws), self._ptrs(ws),
                                                    self._ptrs(bs), warmup, max_runs, budget_s, _dp(t), self._ptrs(outs))
        return self._times(t, cnt), outs

    def time_linear_backward_layers(self, xs, ws, bs, gs, warmup, max_runs, budget_s):
        dims = [xs[0].shape[1]] + [w.shape[0] for w in ws]
        M = xs[0].shape[0]
        dx = [np.empty_like(x) for x in xs]
        dw = [np.empty_like(w) for w in ws]
        db = [np.empty_like(b) for b in bs]
        t = np.empty(max_runs, np.float64)
        cnt = self.lib.nnref_time_linear_backward_layers(self._ptrs(xs), M, (C.c_size_t * len(dims))(*dims), len(ws),
                                                         self._ptrs(ws), self._ptrs(bs), self._ptrs(gs), warmup,
                                                         max_runs, budget_s, _dp(t), self._ptrs(dx), self._ptrs(dw),
                                                         self._ptrs(db))
        return self._times(t, cnt), [v for i in range(len(ws)) for v in (dx[i], dw[i], db[i])]

    def time_conv2d(self, x, w, bias, stride, pad, fuse_relu, g, warmup, max_runs, budget_s):
        """Forward times and output; then, when g is given, the backward rule's times and (dx, dw, db)."""
        N, Cin, H, W = x.shape
        Cout, _, kh, kw = w.shape
        ho, wo = Oracle.conv_out(H, W, kh, kw, stride, pad)
        y = np.empty((N, Cout, ho, wo), np.float32)
        dx, dw, db = np.empty_like(x), np.empty_like(w), np.empty_like(bias)
        tf, tb = np.empty(max_runs, np.float64), np.empty(max_runs, np.float64)
        nf = C.c_int(0)
        nb = self.lib.nnref_time_conv2d(_fp(x), N, Cin, H, W, _fp(w), Cout, kh, kw, _fp(bias), stride, pad,
                                        int(fuse_relu), _fp(g) if g is not None else None, warmup, max_runs, budget_s,
                                        _dp(tf), C.byref(nf), _dp(tb), _fp(y), _fp(dx), _fp(dw), _fp(db))
        fwd = (self._times(tf, nf.value), y)
        bwd = (self._times(tb, nb), (dx, dw, db)) if g is not None else None
        return fwd, bwd

    def time_maxpool2d(self, x, k, s, g, warmup, max_runs, budget_s):
        N, Cc, H, W = x.shape
        y = np.empty((N, Cc, (H - k) // s + 1, (W - k) // s + 1), np.float32)
        dx = np.empty_like(x)
        tf, tb = np.empty(max_runs, np.float64), np.empty(max_runs, np.float64)
        nf = C.c_int(0)
        nb = self.lib.nnref_time_maxpool2d(_fp(x), N, Cc, H, W, k, s, _fp(g), warmup, max_runs, budget_s, _dp(tf),
                                           C.byref(nf), _dp(tb), _fp(y), _fp(dx))
        return (self._times(tf, nf.value), y), (self._times(tb, nb), dx)

    def time_batchnorm(self, x, w, b, eps, relu, g, warmup, max_runs, budget_s):
        N, Cc, S = Oracle._nsc(x)
        y, dx = np.empty_like(x), np.empty_like(x)
        tf, tb = np.empty(max_runs, np.float64), np.empty(max_runs, np.float64)
        nf = C.c_int(0)
        nb = self.lib.nnref_time_batchnorm(_fp(x), N, Cc, S, _fp(w), _fp(b), float(eps), int(relu), _fp(g), warmup,
                                           max_runs, budget_s, _dp(tf), C.byref(nf), _dp(tb), _fp(y), _fp(dx))
        return (self._times(tf, nf.value), y), (self._times(tb, nb), dx)

    def time_layernorm(self, x, gamma, beta, eps, g, warmup, max_runs, budget_s):
        D = x.shape[-1]
        y, dx = np.empty_like(x), np.empty_like(x)
        tf, tb = np.empty(max_runs, np.float64), np.empty(max_runs, np.float64)
        nf = C.c_int(0)
        nb = self.lib.nnref_time_layernorm(_fp(x), x.size // D, D, _fp(gamma), _fp(beta), float(eps), _fp(g), warmup,
                                           max_runs, budget_s, _dp(tf), C.byref(nf), _dp(tb), _fp(y), _fp(dx))
        return (self._times(tf, nf.value), y), (self._times(tb, nb), dx)

    def time_attention(self, q, k, v, heads, causal, g, warmup, max_runs, budget_s):
        N, T, D = q.shape
        out, dq, dk, dv = np.empty_like(q), np.empty_like(q), np.empty_like(k), np.empty_like(v)
        tf, tb = np.empty(max_runs, np.float64), np.empty(max_runs, np.float64)
        nf = C.c_int(0)
        nb = self.lib.nnref_time_attention(_fp(q), _fp(k), _fp(v), N, T, D, heads, int(causal),
                                           _fp(g) if g is not None else None, warmup, max_runs, budget_s, _dp(tf),
                                           C.byref(nf), _dp(tb), _fp(out), _fp(dq), _fp(dk), _fp(dv))
        fwd = (self._times(tf, nf.value), out)
        bwd = (self._times(tb, nb), (dq, dk, dv)) if g is not None else None
        return fwd, bwd


def reference_available():
    return os.path.exists(REF_SO)

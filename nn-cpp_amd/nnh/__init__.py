"""Python binding of libnnh (include/nnh.h) for tests and benchmarks.

The product is the C ABI in lib/libnnh.so; this module only loads it with ctypes and passes device
pointers of torch tensors (torch is used for device memory and streams). Every call raises NnhError
(ShapeError for nn-cpp's TensorShapeError) when the library returns a non-zero status, and the module
refuses to run at all when the library is missing: there is no fallback path.
"""
import ctypes as C
import os

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_ROOT, "lib", "libnnh.so")
HOST_LIB_PATH = os.path.join(PKG_ROOT, "lib", "libnn_gemm_hip.so")
BENCH_LIB_PATH = os.path.join(PKG_ROOT, "lib", "libnnh_bench.so")
REPO_ROOT = os.path.dirname(PKG_ROOT)
HEADER_PATH = os.path.join(REPO_ROOT, "include", "nnh.h")

OK, ERR_INVALID, ERR_SHAPE, ERR_ALIAS, ERR_HIP, ERR_WORKSPACE = 0, 1, 2, 3, 4, 5
NUMERICS_DEFAULT, NUMERICS_NNCPP, NUMERICS_SPLIT_DEPTH = -1, 0, 1
BIAS_NONE, BIAS_COL, BIAS_ROW = 0, 1, 2
MAX_BATCH_DIMS = 4


class NnhError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"nnh error {code}: {msg}")
        self.code = code


class ShapeError(NnhError):
    """nn-cpp's TensorShapeError."""


class Batch(C.Structure):
    _fields_ = [("ndim", C.c_int), ("shape", C.c_size_t * MAX_BATCH_DIMS),
                ("stride_a", C.c_ssize_t * MAX_BATCH_DIMS), ("stride_b", C.c_ssize_t * MAX_BATCH_DIMS),
                ("stride_c", C.c_ssize_t * MAX_BATCH_DIMS)]


class Epilogue(C.Structure):
    _fields_ = [("bias_mode", C.c_int), ("relu", C.c_int), ("bias", C.c_void_p), ("alive", C.c_void_p)]


_lib = None
_sz = C.c_size_t
_vp = C.c_void_p
_szp = C.POINTER(C.c_size_t)


def _declare(L):
    gemm = [C.c_int, C.c_int, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _vp, _sz, C.c_int]
    L.nnh_last_error.restype = C.c_char_p
    L.nnh_version.restype = C.c_char_p
    L.nnh_sgemm.argtypes = gemm + [_vp]
    L.nnh_sgemm_batched.argtypes = gemm + [C.POINTER(Batch), C.POINTER(Epilogue), _vp]
    L.nnh_sgemm_config.argtypes = gemm + [C.POINTER(Batch), C.POINTER(Epilogue), C.c_int, _vp]
    L.nnh_gemm_config_name.restype = C.c_char_p
    L.nnh_matmul_shape.argtypes = [_szp, C.c_int, _szp, C.c_int, C.c_int, C.c_int, _szp, C.POINTER(C.c_int)]
    L.nnh_matmul.argtypes = [_vp, _szp, C.c_int, _vp, _szp, C.c_int, C.c_int, C.c_int, _vp, _vp]
    for name, args in _EXTRA_DECLS.items():
        if hasattr(L, name):
            getattr(L, name).argtypes = args
    if hasattr(L, "nnh_sgemm_noalloc_max_workspace"):
        L.nnh_sgemm_noalloc_max_workspace.restype = _sz


_EXTRA_DECLS = {
    "nnh_linear_forward": [_vp, _sz, _sz, _vp, _sz, _vp, C.c_int, _vp, _vp],
    "nnh_linear_backward": [_vp, _vp, _vp, _szp, C.c_int, _sz, _sz, _vp, C.c_int, _vp, C.c_int, _vp, C.c_int, _vp],
    "nnh_relu_forward": [_vp, _vp, _sz, _vp],
    "nnh_relu_backward": [_vp, _vp, _vp, C.c_int, _sz, _vp],
    "nnh_tensor_sum0": [_vp, _sz, _sz, _vp, C.c_int, _vp],
    "nnh_zero_many": [_vp, _vp, _sz, _vp],
    "nnh_attention_forward": [_vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _vp, C.c_int, _vp, _vp, _vp],
    "nnh_attention_backward": [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _vp, C.c_int, _vp, C.c_int, _vp,
                               C.c_int, _vp, C.c_int, _vp],
    "nnh_scaled_masked_softmax_forward": [_vp, _sz, _sz, _sz, _sz, C.c_float, _vp, C.c_int, _vp, _vp],
    "nnh_scaled_masked_softmax_backward": [_vp, _vp, _sz, _sz, _sz, _sz, C.c_float, _vp, C.c_int, _vp, C.c_int, _vp],
    "nnh_conv2d_forward": [_vp, _sz, _sz, _sz, _sz, _vp, _sz, _sz, _sz, _vp, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp],
    "nnh_conv2d_backward": [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _sz, C.c_int, C.c_int, _vp, C.c_int,
                            _vp, C.c_int, _vp, C.c_int, _vp],
    "nnh_set_workspace": [_vp, _vp, _sz],
    "nnh_sgemm_workspace_size": [_sz, _sz, _sz, _sz, _szp],
    "nnh_matmul_workspace_size": [_szp, C.c_int, _szp, C.c_int, C.c_int, C.c_int, _szp],
    "nnh_linear_forward_workspace_size": [_sz, _sz, _sz, _szp],
    "nnh_linear_backward_workspace_size": [_szp, C.c_int, _sz, _sz, C.c_int, C.c_int, C.c_int, _szp],
    "nnh_conv2d_forward_workspace_size": [_sz, _sz, _sz, _sz, _sz, _sz, _sz, C.c_int, C.c_int, _szp],
    "nnh_conv2d_backward_workspace_size": [_sz, _sz, _sz, _sz, _sz, _sz, _sz, C.c_int, C.c_int, C.c_int, C.c_int,
                                           C.c_int, C.c_int, _szp],
    "nnh_attention_forward_workspace_size": [_sz, _sz, _sz, _sz, _sz, _szp],
    "nnh_attention_backward_workspace_size": [_sz, _sz, _sz, _sz, _sz, _szp],
    "nnh_sgemm_noalloc": [C.c_int, C.c_int, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _vp, _sz, C.c_int, _vp],
    "nnh_maxpool2d_forward": [_vp, _sz, _sz, _sz, _sz, _sz, _sz, _vp, _vp, _vp],
    "nnh_conv2d_relu_maxpool2d_forward": [_vp, _sz, _sz, _sz, _sz, _vp, _sz, _sz, _sz, _vp, C.c_int, C.c_int, _sz, _sz,
                                          _vp, _vp, _vp, _vp, _vp],
    "nnh_maxpool2d_backward": [_vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _vp, C.c_int, _vp],
    "nnh_conv2d_packed_supported": [_sz, _sz, _sz, _sz, _sz, _sz, _sz, C.c_int, C.c_int, C.c_int],
    "nnh_conv2d_relu_forward_packed": [_vp, _sz, _sz, _sz, _sz, _vp, _sz, _sz, _sz, _vp, C.c_int, C.c_int, _vp, _vp,
                                       _vp],
    "nnh_conv2d_relu_maxpool2d_forward_packed": [_vp, _sz, _sz, _sz, _sz, _vp, _sz, _sz, _sz, _vp, C.c_int, C.c_int,
                                                 _vp, _vp, _vp, _vp, _vp],
    "nnh_conv2d_backward_packed": [_vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _sz, _sz, _sz, C.c_int, C.c_int, _vp,
                                   C.c_int, _vp, C.c_int, _vp, C.c_int, _vp],
    "nnh_maxpool2d_backward_packed": [_vp, _vp, _sz, _sz, _sz, _sz, _vp, C.c_int, _vp],
    "nnh_matmul_backward": [_vp, _vp, _szp, C.c_int, _vp, _szp, C.c_int, C.c_int, _vp, C.c_int, _vp, C.c_int, _vp],
    "nnh_matmul_backward_workspace_size": [_szp, C.c_int, _szp, C.c_int, C.c_int, C.c_int, C.c_int, _szp],
    "nnh_add_to_grad": [_vp, _vp, _sz, C.c_int, _vp],
    "nnh_add_to_grad2": [_vp, C.c_int, _vp, C.c_int, _vp, _sz, _vp],
    "nnh_linear_forward_add": [_vp, _sz, _sz, _vp, _sz, _vp, _vp, _vp, _vp],
    "nnh_linear_gelu_forward": [_vp, _sz, _sz, _vp, _sz, _vp, _vp, _vp, _vp, _vp],
    "nnh_embedding_add_forward": [_vp, _sz, _sz, _vp, _sz, _vp, _sz, _vp, _vp],
    "nnh_linear_forward_multi": [_vp, _sz, _sz, C.c_int, C.POINTER(_vp), _szp, C.POINTER(_vp), C.POINTER(_vp), _vp],
    "nnh_im2col": [_vp, _sz, _sz, _sz, _sz, _sz, _sz, C.c_int, C.c_int, _vp, _vp],
    "nnh_col2im_add": [_vp, _sz, _sz, _sz, _sz, _sz, _sz, C.c_int, C.c_int, _vp, C.c_int, _vp],
    "nnh_batchnorm_forward": [_vp, _sz, _sz, _sz, _vp, _vp, C.c_float, C.c_int, _vp, _vp, _vp, _vp, _vp, _vp],
    "nnh_batchnorm_backward": [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _vp, C.c_int, _vp, C.c_int, _vp, C.c_int,
                               _vp],
    "nnh_batchnorm_workspace_size": [_sz, _sz, _sz, _szp],
    "nnh_layernorm_forward": [_vp, _sz, _sz, _vp, _vp, C.c_float, _vp, _vp, _vp, _vp],
    "nnh_layernorm_backward": [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _vp, C.c_int, _vp, C.c_int, _vp, C.c_int, _vp],
    "nnh_add_forward": [_vp, _vp, _sz, _sz, _vp, _vp],
    "nnh_mul_forward": [_vp, _vp, _sz, _vp, _vp],
    "nnh_mul_backward": [_vp, _vp, _sz, _vp, C.c_int, _vp],
    "nnh_gelu_forward": [_vp, _sz, _vp, _vp, _vp],
    "nnh_gelu_backward": [_vp, _vp, _vp, _sz, _vp, C.c_int, _vp],
    "nnh_embedding_forward": [_vp, _sz, _sz, _vp, _sz, _vp, _vp],
    "nnh_embedding_backward": [_vp, _vp, _sz, _sz, _sz, _vp, C.c_int, _vp],
    "nnh_set_stream_numerics": [_vp, C.c_int],
    "nnh_get_stream_numerics": [_vp],
}


def set_numerics(mode):
    """NUMERICS_NNCPP (nn-cpp's bits) or NUMERICS_SPLIT_DEPTH (128-deep chains for small products); returns the
    previous mode."""
    prev = lib().nnh_get_numerics()
    check(lib().nnh_set_numerics(int(mode)))
    return prev


def set_stream_numerics(mode, stream=None):
    """The mode of every call on `stream` (torch's current stream by default); NUMERICS_DEFAULT clears it, and the
    stream follows the process default again."""
    check(lib().nnh_set_stream_numerics(_stream(stream), int(mode)))


def get_stream_numerics(stream=None):
    return lib().nnh_get_stream_numerics(_stream(stream))


def workspace_size(name, *args):
    """Bytes of scratch the call nnh_<name> takes, from its nnh_<name>_workspace_size query (the call's shape
    arguments; a list or tuple becomes a size_t array)."""
    conv = []
    for a in args:
        if isinstance(a, (list, tuple)):
            conv.append((C.c_size_t * max(1, len(a)))(*a))
        else:
            conv.append(a)
    out = C.c_size_t(0)
    check(getattr(lib(), f"nnh_{name}_workspace_size")(*conv, C.byref(out)))
    return out.value


def set_workspace(buf, stream=None):
    """Registers the device tensor buf as the scratch of every call on stream (None: the library owns it again)."""
    if buf is None:
        check(lib().nnh_set_workspace(_stream(stream), None, 0))
    else:
        check(lib().nnh_set_workspace(_stream(stream), C.c_void_p(buf.data_ptr()), buf.numel() * buf.element_size()))


def lib():
    """The loaded library; raises if it has not been built (no fallback exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C nn-cpp_amd` "
                               "(or __graft_entry__.build()); nnh has no CPU fallback")
        L = C.CDLL(LIB_PATH)
        _declare(L)
        _lib = L
    return _lib


def check(rc):
    if rc != OK:
        msg = lib().nnh_last_error().decode()
        raise (ShapeError if rc == ERR_SHAPE else NnhError)(rc, msg)


def header_functions():
    """Names of every function the headers of libnnh declare (include/nnh*.h except nnh_host.h, which belongs to
    the drop-in library)."""
    import glob
    import re
    names = set()
    for path in glob.glob(os.path.join(os.path.dirname(HEADER_PATH), "nnh*.h")):
        if os.path.basename(path) != "nnh_host.h":
            names |= set(re.findall(r"\b(nnh_[a-z0-9_]+)\s*\(", open(path).read()))
    return sorted(names)


# ---- torch plumbing ----

def _stream(stream):
    import torch
    if stream is None:
        stream = torch.cuda.current_stream()
    return C.c_void_p(stream.cuda_stream)


def _ptr(t, offset=0):
    if t is None:
        return None
    import torch
    assert t.dtype in (torch.float32, torch.uint8, torch.int32), t.dtype
    assert t.is_cuda, "nnh works on device tensors"
    return C.c_void_p(t.data_ptr() + offset * t.element_size())


def make_batch(shape=(), sa=(), sb=(), sc=()):
    b = Batch()
    b.ndim = len(shape)
    for i, d in enumerate(shape):
        b.shape[i], b.stride_a[i], b.stride_b[i], b.stride_c[i] = d, sa[i], sb[i], sc[i]
    return b


def make_epilogue(bias_mode=BIAS_NONE, bias=None, relu=False, alive=None):
    e = Epilogue()
    e.bias_mode = bias_mode
    e.relu = int(bool(relu))
    e.bias = _ptr(bias).value if bias is not None else None
    e.alive = _ptr(alive).value if alive is not None else None
    return e


def sgemm(ta, tb, m, n, k, a, lda, b, ldb, c, ldc, accumulate=False, stream=None):
    """nn::kernels::sgemm on device tensors a, b, c (their first element is the matrix origin)."""
    check(lib().nnh_sgemm(int(ta), int(tb), m, n, k, _ptr(a), lda, _ptr(b), ldb, _ptr(c), ldc, int(accumulate),
                          _stream(stream)))


def sgemm_batched(ta, tb, m, n, k, a, lda, b, ldb, c, ldc, accumulate=False, batch=None, epilogue=None,
                  config=-1, stream=None):
    bp = C.byref(batch) if batch is not None else None
    ep = C.byref(epilogue) if epilogue is not None else None
    check(lib().nnh_sgemm_config(int(ta), int(tb), m, n, k, _ptr(a), lda, _ptr(b), ldb, _ptr(c), ldc,
                                 int(accumulate), bp, ep, int(config), _stream(stream)))


def gemm_configs():
    L = lib()
    return [L.nnh_gemm_config_name(i).decode() for i in range(L.nnh_gemm_config_count())]


def matmul_shape(a_shape, b_shape, ta=False, tb=False):
    ash = (C.c_size_t * max(1, len(a_shape)))(*a_shape)
    bsh = (C.c_size_t * max(1, len(b_shape)))(*b_shape)
    out = (C.c_size_t * 16)()
    nd = C.c_int(0)
    check(lib().nnh_matmul_shape(ash, len(a_shape), bsh, len(b_shape), int(ta), int(tb), out, C.byref(nd)))
    return tuple(out[i] for i in range(nd.value))


def matmul(a, b, ta=False, tb=False, stream=None):
    """nn::matmul(a, b, ta, tb) on contiguous device tensors; returns a new tensor."""
    import torch
    assert a.is_contiguous() and b.is_contiguous()
    shape = matmul_shape(a.shape, b.shape, ta, tb)
    out = torch.empty(shape, dtype=torch.float32, device=a.device)
    ash = (C.c_size_t * a.dim())(*a.shape)
    bsh = (C.c_size_t * b.dim())(*b.shape)
    check(lib().nnh_matmul(_ptr(a), ash, a.dim(), _ptr(b), bsh, b.dim(), int(ta), int(tb), _ptr(out),
                           _stream(stream)))
    return out


def matmul_backward(g, a, b, b_transposed=False, da=None, da_first=True, db=None, db_first=True, stream=None):
    """nn::matmul / nn::matmul_bt backward into the given gradient buffers (either may be None)."""
    ash = (C.c_size_t * a.dim())(*a.shape)
    bsh = (C.c_size_t * b.dim())(*b.shape)
    check(lib().nnh_matmul_backward(_ptr(g), _ptr(a), ash, a.dim(), _ptr(b), bsh, b.dim(), int(b_transposed), _ptr(da),
                                    int(da_first), _ptr(db), int(db_first), _stream(stream)))


def linear_forward(x, w, bias, relu=False, stream=None):
    """nn::linear (optionally followed by nn::relu) on device tensors; returns y."""
    import torch
    K = x.shape[-1]
    M = x.numel() // K if K else int(torch.tensor(x.shape[:-1]).prod())
    n = w.shape[0]
    y = torch.empty(tuple(x.shape[:-1]) + (n,), dtype=torch.float32, device=x.device)
    check(lib().nnh_linear_forward(_ptr(x), M, K, _ptr(w), n, _ptr(bias), int(relu), _ptr(y), _stream(stream)))
    return y


def linear_forward_multi(x, layers, stream=None):
    """Several nn::linear forwards over one input x; layers is [(w, bias), ...]; returns the outputs."""
    import torch
    K = x.shape[-1]
    M = x.numel() // K if K else int(torch.tensor(x.shape[:-1]).prod())
    ys = [torch.empty(tuple(x.shape[:-1]) + (w.shape[0],), dtype=torch.float32, device=x.device) for w, _ in layers]
    cnt = len(layers)
    arr = lambda ts: (_vp * cnt)(*[t.data_ptr() for t in ts])
    ns = (C.c_size_t * cnt)(*[w.shape[0] for w, _ in layers])
    check(lib().nnh_linear_forward_multi(_ptr(x), M, K, cnt, arr([w for w, _ in layers]), ns,
                                         arr([b for _, b in layers]), arr(ys), _stream(stream)))
    return ys


def linear_forward_add(x, w, bias, residual, out=None, stream=None):
    """nn::add(residual, nn::linear(x, w, bias)) in one kernel; returns y (out, which may be residual itself)."""
    import torch
    K = x.shape[-1]
    M = x.numel() // K if K else int(torch.tensor(x.shape[:-1]).prod())
    n = w.shape[0]
    y = out if out is not None else torch.empty(tuple(x.shape[:-1]) + (n,), dtype=torch.float32, device=x.device)
    check(lib().nnh_linear_forward_add(_ptr(x), M, K, _ptr(w), n, _ptr(bias), _ptr(residual), _ptr(y),
                                       _stream(stream)))
    return y


def linear_backward(g, x, w, dx=None, dx_first=True, dw=None, dw_first=True, db=None, db_first=True, stream=None):
    """nn::linear's backward into the given gradient buffers (any may be None)."""
    lead = (C.c_size_t * (x.dim() - 1))(*x.shape[:-1])
    check(lib().nnh_linear_backward(_ptr(g), _ptr(x), _ptr(w), lead, x.dim() - 1, x.shape[-1], w.shape[0],
                                    _ptr(dx), int(dx_first), _ptr(dw), int(dw_first), _ptr(db), int(db_first),
                                    _stream(stream)))


def relu_forward(x, stream=None):
    import torch
    y = torch.empty_like(x)
    check(lib().nnh_relu_forward(_ptr(x), _ptr(y), x.numel(), _stream(stream)))
    return y


def relu_backward(x, g, dx, first=True, stream=None):
    check(lib().nnh_relu_backward(_ptr(x), _ptr(g), _ptr(dx), int(first), x.numel(), _stream(stream)))


def tensor_sum0(src, dst, combine=0, stream=None):
    rows = src.shape[0]
    inner = src.numel() // rows if rows else dst.numel()
    check(lib().nnh_tensor_sum0(_ptr(src), rows, inner, _ptr(dst), int(combine), _stream(stream)))


def zero_many(tensors, stream=None):
    """Every float32 device tensor in `tensors` filled with +0 in one launch per 32 (nnh_zero_many)."""
    import torch
    for t in tensors:
        assert t.dtype == torch.float32 and t.is_cuda and t.is_contiguous(), "zero_many takes contiguous float32 device tensors"
    ptrs = (C.c_void_p * max(1, len(tensors)))(*[t.data_ptr() for t in tensors])
    counts = (C.c_size_t * max(1, len(tensors)))(*[t.numel() for t in tensors])
    check(lib().nnh_zero_many(C.cast(ptrs, C.c_void_p), C.cast(counts, C.c_void_p), len(tensors), _stream(stream)))


def attention_forward(q, k, v, heads, mask=None, causal=False, stream=None):
    """nn::attention forward on device tensors; returns (out, probs)."""
    import torch
    N, Tq, D = q.shape
    Tk = k.shape[1]
    out = torch.empty((N, Tq, D), dtype=torch.float32, device=q.device)
    probs = torch.empty((N, heads, Tq, Tk), dtype=torch.float32, device=q.device)
    check(lib().nnh_attention_forward(_ptr(q), _ptr(k), _ptr(v), N, Tq, Tk, D, heads, _ptr(mask), int(causal),
                                      _ptr(out), _ptr(probs), _stream(stream)))
    return out, probs


def attention_backward(g, q, k, v, probs, heads, mask=None, causal=False, dq=None, dq_first=True, dk=None,
                       dk_first=True, dv=None, dv_first=True, stream=None):
    N, Tq, D = q.shape
    Tk = k.shape[1]
    check(lib().nnh_attention_backward(_ptr(g), _ptr(q), _ptr(k), _ptr(v), _ptr(probs), N, Tq, Tk, D, heads,
                                       _ptr(mask), int(causal), _ptr(dq), int(dq_first), _ptr(dk), int(dk_first),
                                       _ptr(dv), int(dv_first), _stream(stream)))


def scaled_masked_softmax_forward(x, scale, mask=None, causal=False, stream=None):
    import torch
    N, H, Tq, Tk = x.shape
    y = torch.empty_like(x)
    check(lib().nnh_scaled_masked_softmax_forward(_ptr(x), N, H, Tq, Tk, float(scale), _ptr(mask), int(causal),
                                                  _ptr(y), _stream(stream)))
    return y


def scaled_masked_softmax_backward(y, g, dx, scale, mask=None, causal=False, first=True, stream=None):
    N, H, Tq, Tk = y.shape
    check(lib().nnh_scaled_masked_softmax_backward(_ptr(y), _ptr(g), N, H, Tq, Tk, float(scale), _ptr(mask),
                                                   int(causal), _ptr(dx), int(first), _stream(stream)))


def conv_out(H, W, kh, kw, stride, pad):
    """conv2d_output_size (ops.cpp:135-139); (0, 0) for geometry the library rejects."""
    if stride <= 0 or pad < 0 or kh > H + 2 * pad or kw > W + 2 * pad:
        return 0, 0
    return (H + 2 * pad - kh) // stride + 1, (W + 2 * pad - kw) // stride + 1


def conv2d_forward(x, w, bias, stride, pad, fuse_relu, want_alive=True, stream=None):
    """nn::conv2d (fuse_relu=False) or nn::conv2d_relu; returns (y, alive or None)."""
    import torch
    N, Cin, H, W = x.shape
    Cout, _, kh, kw = w.shape
    ho, wo = conv_out(H, W, kh, kw, stride, pad)
    y = torch.empty((N, Cout, max(ho, 0), max(wo, 0)), dtype=torch.float32, device=x.device)
    alive = torch.empty(y.shape, dtype=torch.uint8, device=x.device) if (fuse_relu and want_alive) else None
    check(lib().nnh_conv2d_forward(_ptr(x), N, Cin, H, W, _ptr(w), Cout, kh, kw, _ptr(bias), int(stride), int(pad),
                                   int(fuse_relu), _ptr(y), _ptr(alive), _stream(stream)))
    return y, alive


def maxpool2d_forward(x, kernel, stride, want_argmax=True, stream=None):
    """nn::maxpool2d on a device tensor {N, C, H, W}; returns (y, argmax or None), argmax as int32 holding the uint32
    offsets inside each (n, c) plane."""
    import torch
    N, Cc, H, W = x.shape
    ho, wo = (H - kernel) // stride + 1, (W - kernel) // stride + 1
    y = torch.empty((N, Cc, ho, wo), dtype=torch.float32, device=x.device)
    argmax = torch.empty(y.shape, dtype=torch.int32, device=x.device) if want_argmax else None
    check(lib().nnh_maxpool2d_forward(_ptr(x), N, Cc, H, W, kernel, stride, _ptr(y), _ptr(argmax), _stream(stream)))
    return y, argmax


def conv2d_relu_maxpool2d_forward(x, w, bias, stride, pad, pool_kernel, pool_stride, want_alive=True,
                                  want_argmax=True, stream=None):
    """nn::conv2d_relu then nn::maxpool2d on its output in one call; returns (y, alive or None, pooled, argmax or
    None), argmax as int32 holding the uint32 offsets."""
    import torch
    N, Cin, H, W = x.shape
    Cout, _, kh, kw = w.shape
    ho, wo = conv_out(H, W, kh, kw, stride, pad)
    y = torch.empty((N, Cout, max(ho, 0), max(wo, 0)), dtype=torch.float32, device=x.device)
    alive = torch.empty(y.shape, dtype=torch.uint8, device=x.device) if want_alive else None
    po, qo = (max(ho - pool_kernel, -1) // pool_stride + 1, max(wo - pool_kernel, -1) // pool_stride + 1) \
        if pool_kernel and pool_stride else (0, 0)
    pooled = torch.empty((N, Cout, max(po, 0), max(qo, 0)), dtype=torch.float32, device=x.device)
    argmax = torch.empty(pooled.shape, dtype=torch.int32, device=x.device) if want_argmax else None
    check(lib().nnh_conv2d_relu_maxpool2d_forward(_ptr(x), N, Cin, H, W, _ptr(w), Cout, kh, kw, _ptr(bias), int(stride),
                                                  int(pad), pool_kernel, pool_stride, _ptr(y), _ptr(alive),
                                                  _ptr(pooled), _ptr(argmax), _stream(stream)))
    return y, alive, pooled, argmax


def conv2d_backward(g, x, w, alive, stride, pad, dx=None, dx_first=True, dw=None, dw_first=True, db=None,
                    db_first=True, stream=None):
    N, Cin, H, W = x.shape
    Cout, _, kh, kw = w.shape
    check(lib().nnh_conv2d_backward(_ptr(g), _ptr(x), _ptr(w), _ptr(alive), N, Cin, H, W, Cout, kh, kw, int(stride),
                                    int(pad), _ptr(dx), int(dx_first), _ptr(dw), int(dw_first), _ptr(db),
                                    int(db_first), _stream(stream)))


def conv2d_packed_supported(x_shape, w_shape, stride, pad, with_pool=False):
    """Whether nnh_conv2d_*_packed take this geometry (pointer alignment is the caller's part)."""
    N, Cin, H, W = x_shape
    Cout, _, kh, kw = w_shape
    return bool(lib().nnh_conv2d_packed_supported(N, Cin, H, W, Cout, kh, kw, int(stride), int(pad), int(with_pool)))


def conv2d_relu_forward_packed(x, w, bias, stride, pad, stream=None):
    """nn::conv2d_relu with its flags packed one bit per output; returns (y, alive_bits as uint8)."""
    import torch
    N, Cin, H, W = x.shape
    Cout, _, kh, kw = w.shape
    ho, wo = conv_out(H, W, kh, kw, stride, pad)
    y = torch.empty((N, Cout, max(ho, 0), max(wo, 0)), dtype=torch.float32, device=x.device)
    bits = torch.empty(((y.numel() + 7) // 8,), dtype=torch.uint8, device=x.device)
    check(lib().nnh_conv2d_relu_forward_packed(_ptr(x), N, Cin, H, W, _ptr(w), Cout, kh, kw, _ptr(bias), int(stride),
                                               int(pad), _ptr(y), _ptr(bits), _stream(stream)))
    return y, bits


def conv2d_relu_maxpool2d_forward_packed(x, w, bias, stride, pad, stream=None):
    """nn::conv2d_relu then a 2 x 2 stride-2 nn::maxpool2d, flags as bits and window maxima as 2-bit positions;
    returns (y, alive_bits, pooled, argmax2), both packed arrays uint8."""
    import torch
    N, Cin, H, W = x.shape
    Cout, _, kh, kw = w.shape
    ho, wo = conv_out(H, W, kh, kw, stride, pad)
    y = torch.empty((N, Cout, max(ho, 0), max(wo, 0)), dtype=torch.float32, device=x.device)
    bits = torch.empty(((y.numel() + 7) // 8,), dtype=torch.uint8, device=x.device)
    pooled = torch.empty((N, Cout, max(ho, 0) // 2, max(wo, 0) // 2), dtype=torch.float32, device=x.device)
    amax2 = torch.empty((N * Cout * (max(ho, 0) // 2) * ((max(wo, 0) + 7) // 8),), dtype=torch.uint8, device=x.device)
    check(lib().nnh_conv2d_relu_maxpool2d_forward_packed(_ptr(x), N, Cin, H, W, _ptr(w), Cout, kh, kw, _ptr(bias),
                                                         int(stride), int(pad), _ptr(y), _ptr(bits), _ptr(pooled),
                                                         _ptr(amax2), _stream(stream)))
    return y, bits, pooled, amax2


def conv2d_backward_packed(g, x, w, alive_bits, stride, pad, dx=None, dx_first=True, dw=None, dw_first=True, db=None,
                           db_first=True, stream=None):
    N, Cin, H, W = x.shape
    Cout, _, kh, kw = w.shape
    check(lib().nnh_conv2d_backward_packed(_ptr(g), _ptr(x), _ptr(w), _ptr(alive_bits), N, Cin, H, W, Cout, kh, kw,
                                           int(stride), int(pad), _ptr(dx), int(dx_first), _ptr(dw), int(dw_first),
                                           _ptr(db), int(db_first), _stream(stream)))


def maxpool2d_backward_packed(g, argmax2, dx, first=True, stream=None):
    """nn::maxpool2d's backward (kernel 2, stride 2) from 2-bit window positions into dx {N, C, H, W}."""
    N, Cc, H, W = dx.shape
    check(lib().nnh_maxpool2d_backward_packed(_ptr(g), _ptr(argmax2), N, Cc, H, W, _ptr(dx), int(first),
                                              _stream(stream)))


def im2col(x, kh, kw, stride, pad, stream=None):
    import torch
    N, Cin, H, W = x.shape
    ho, wo = conv_out(H, W, kh, kw, stride, pad)
    col = torch.empty((N, Cin * kh * kw, ho * wo), dtype=torch.float32, device=x.device)
    check(lib().nnh_im2col(_ptr(x), N, Cin, H, W, kh, kw, int(stride), int(pad), _ptr(col), _stream(stream)))
    return col


def col2im_add(col, dx, kh, kw, stride, pad, first=False, stream=None):
    N, Cin, H, W = dx.shape
    check(lib().nnh_col2im_add(_ptr(col), N, Cin, H, W, kh, kw, int(stride), int(pad), _ptr(dx), int(first),
                               _stream(stream)))


def batchnorm_forward(x, weight, bias, eps, fuse_relu=False, want_alive=True, stream=None):
    """nn::batchnorm (training mode) on a device tensor {N, C, ...}; returns (y, alive or None, mean, var, inv_std)."""
    import torch
    N, Cc = x.shape[0], x.shape[1]
    S = 1
    for d in x.shape[2:]:
        S *= d
    y = torch.empty_like(x)
    alive = torch.empty(x.shape, dtype=torch.uint8, device=x.device) if (fuse_relu and want_alive) else None
    mean, var, inv = (torch.empty(Cc, dtype=torch.float32, device=x.device) for _ in range(3))
    check(lib().nnh_batchnorm_forward(_ptr(x), N, Cc, S, _ptr(weight), _ptr(bias), float(eps), int(fuse_relu), _ptr(y),
                                      _ptr(alive), _ptr(mean), _ptr(var), _ptr(inv), _stream(stream)))
    return y, alive, mean, var, inv


def batchnorm_backward(g, x, alive, weight, mean, inv_std, dx=None, dx_first=True, dw=None, dw_first=True, db=None,
                       db_first=True, stream=None):
    N, Cc = x.shape[0], x.shape[1]
    S = 1
    for d in x.shape[2:]:
        S *= d
    check(lib().nnh_batchnorm_backward(_ptr(g), _ptr(x), _ptr(alive), _ptr(weight), _ptr(mean), _ptr(inv_std), N, Cc,
                                       S, _ptr(dx), int(dx_first), _ptr(dw), int(dw_first), _ptr(db), int(db_first),
                                       _stream(stream)))


def layernorm_forward(x, gamma, beta, eps, stream=None):
    """nn::layernorm over the last axis of a device tensor; returns (y, mean, inv_std), one statistic per row."""
    import torch
    D = x.shape[-1]
    R = x.numel() // D
    y = torch.empty_like(x)
    mean = torch.empty(R, dtype=torch.float32, device=x.device)
    inv = torch.empty(R, dtype=torch.float32, device=x.device)
    check(lib().nnh_layernorm_forward(_ptr(x), R, D, _ptr(gamma), _ptr(beta), float(eps), _ptr(y), _ptr(mean),
                                      _ptr(inv), _stream(stream)))
    return y, mean, inv


def layernorm_backward(g, x, gamma, mean, inv_std, dx=None, dx_first=True, dgamma=None, dgamma_first=True,
                       dbeta=None, dbeta_first=True, stream=None):
    D = x.shape[-1]
    R = x.numel() // D
    check(lib().nnh_layernorm_backward(_ptr(g), _ptr(x), _ptr(gamma), _ptr(mean), _ptr(inv_std), R, D, _ptr(dx),
                                       int(dx_first), _ptr(dgamma), int(dgamma_first), _ptr(dbeta), int(dbeta_first),
                                       _stream(stream)))


_bench_lib = None


def bench_delay(microseconds, stream=None):
    """Occupies the stream for `microseconds` of device time (libnnh_bench.so, a measurement helper): calls
    queued behind it then run back to back, so events around them time the device, not the Python caller."""
    global _bench_lib
    if _bench_lib is None:
        if not os.path.exists(BENCH_LIB_PATH):
            raise RuntimeError(f"{BENCH_LIB_PATH} is missing: build it with `make -C nn-cpp_amd`")
        L = C.CDLL(BENCH_LIB_PATH)
        L.nnh_bench_delay.argtypes = [C.c_double, _vp]
        _bench_lib = L
    rc = _bench_lib.nnh_bench_delay(float(microseconds), _stream(stream))
    if rc != 0:
        raise NnhError(ERR_HIP, f"nnh_bench_delay: HIP error {rc}")


_host_lib = None


def host_lib():
    """libnn_gemm_hip.so: the drop-in nn::kernels::sgemm (host pointers) built on libnnh."""
    global _host_lib
    if _host_lib is None:
        if not os.path.exists(HOST_LIB_PATH):
            raise RuntimeError(f"{HOST_LIB_PATH} is missing: build it with `make -C nn-cpp_amd`")
        L = C.CDLL(HOST_LIB_PATH)
        L.nnh_sgemm_host.argtypes = [C.c_int, C.c_int, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _vp, _sz, C.c_int]
        _host_lib = L
    return _host_lib


def sgemm_host(ta, tb, m, n, k, a, lda, b, ldb, c, ldc, accumulate=False):
    """nn::kernels::sgemm's exact signature on host numpy arrays (C updated in place)."""
    import numpy as np
    for arr in (a, b, c):
        assert arr.dtype == np.float32 and arr.flags["C_CONTIGUOUS"]
    rc = host_lib().nnh_sgemm_host(int(ta), int(tb), m, n, k, a.ctypes.data, lda, b.ctypes.data, ldb, c.ctypes.data,
                                   ldc, int(accumulate))
    if rc != OK:
        raise NnhError(rc, "nn::kernels::sgemm (HIP) failed")

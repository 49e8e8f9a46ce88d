"""The C ABI without a GPU: the library loads, exports every function include/nnh.h declares, and rejects
invalid calls on the host before touching the device (no compute call is made here)."""
import ctypes as C

import pytest

import nnh


def test_library_exports_every_declared_function():
    L = nnh.lib()
    names = nnh.header_functions()
    assert "nnh_sgemm" in names and len(names) >= 8
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_host_library_exports_its_header():
    import re
    text = open(nnh.HEADER_PATH.replace("nnh.h", "nnh_host.h")).read()
    names = sorted(set(re.findall(r"\b(nnh_[a-z0-9_]+)\s*\(", text)))
    L = nnh.host_lib()
    assert names and not [n for n in names if not hasattr(L, n)]


def test_version_and_configs():
    assert b"gfx950" in nnh.lib().nnh_version()
    assert len(nnh.gemm_configs()) >= 1


def _sgemm(*args):
    return nnh.lib().nnh_sgemm(*args)


FAKE_A, FAKE_B, FAKE_C = 0x10000000, 0x20000000, 0x30000000  # host-side address checks only


def test_invalid_arguments_are_rejected_on_the_host():
    L = nnh.lib()
    # null operands with k > 0
    assert _sgemm(0, 0, 4, 4, 4, None, 4, C.c_void_p(FAKE_B), 4, C.c_void_p(FAKE_C), 4, 0, None) == nnh.ERR_INVALID
    assert _sgemm(0, 0, 4, 4, 4, C.c_void_p(FAKE_A), 4, C.c_void_p(FAKE_B), 4, None, 4, 0, None) == nnh.ERR_INVALID
    # leading dimensions too small for the stored layouts
    assert _sgemm(0, 0, 4, 5, 6, C.c_void_p(FAKE_A), 5, C.c_void_p(FAKE_B), 5, C.c_void_p(FAKE_C), 5, 0, None) == nnh.ERR_INVALID
    assert _sgemm(1, 0, 4, 5, 6, C.c_void_p(FAKE_A), 3, C.c_void_p(FAKE_B), 5, C.c_void_p(FAKE_C), 5, 0, None) == nnh.ERR_INVALID
    assert _sgemm(0, 1, 4, 5, 6, C.c_void_p(FAKE_A), 6, C.c_void_p(FAKE_B), 5, C.c_void_p(FAKE_C), 5, 0, None) == nnh.ERR_INVALID
    assert _sgemm(0, 0, 4, 5, 6, C.c_void_p(FAKE_A), 6, C.c_void_p(FAKE_B), 5, C.c_void_p(FAKE_C), 4, 0, None) == nnh.ERR_INVALID
    assert b"ldc" in L.nnh_last_error()
    # sizes beyond the kernel's 32-bit index range
    assert _sgemm(0, 0, 1 << 31, 4, 4, C.c_void_p(FAKE_A), 4, C.c_void_p(FAKE_B), 4, C.c_void_p(FAKE_C), 4, 0, None) == nnh.ERR_INVALID


def test_output_aliasing_an_input_is_rejected():
    """include/nn/kernels/gemm.hpp:37-39: C must not alias A or B."""
    assert _sgemm(0, 0, 4, 4, 4, C.c_void_p(FAKE_A), 4, C.c_void_p(FAKE_B), 4, C.c_void_p(FAKE_A + 16), 4, 0, None) == nnh.ERR_ALIAS
    assert _sgemm(0, 0, 4, 4, 4, C.c_void_p(FAKE_A), 4, C.c_void_p(FAKE_B), 4, C.c_void_p(FAKE_B - 16), 4, 0, None) == nnh.ERR_ALIAS


def test_add_to_grad2_refuses_overlapping_gradients():
    """nnh_add_to_grad2 writes two gradients of one source in one launch: gradients that overlap each other or the
    source are refused on the host (one node passed as both operands takes two nnh_add_to_grad calls)."""
    L = nnh.lib()
    f = L.nnh_add_to_grad2
    a, b, s = C.c_void_p(FAKE_A), C.c_void_p(FAKE_B), C.c_void_p(FAKE_C)
    assert f(a, 1, C.c_void_p(FAKE_A + 16), 0, s, 64, None) == nnh.ERR_ALIAS
    assert f(a, 1, b, 1, C.c_void_p(FAKE_B + 4), 8, None) == nnh.ERR_ALIAS
    assert f(a, 1, None, 1, s, 8, None) == nnh.ERR_INVALID
    assert f(None, 1, None, 1, None, 0, None) == nnh.OK


def test_packed_flag_geometries_on_the_host():
    """nnh_conv2d_packed_supported (no device needed): a first layer's geometry takes the packed flags; stride,
    depth, channel count, plane size and (with the pool) odd heights or rows wider than 256 do not."""
    ok = lambda xs, ws, s=1, p=1, pool=False: nnh.conv2d_packed_supported(xs, ws, s, p, pool)
    assert ok((128, 1, 28, 28), (32, 1, 3, 3)) and ok((128, 1, 28, 28), (32, 1, 3, 3), pool=True)
    assert ok((2, 1, 4, 256), (2, 1, 3, 3), pool=True)
    assert not ok((2, 1, 4, 264), (2, 1, 3, 3), pool=True)      # a row wider than 256
    assert not ok((2, 1, 9, 8), (4, 1, 3, 3), pool=True)        # an odd height
    assert not ok((2, 1, 28, 28), (32, 1, 3, 3), s=2)           # stride 2
    assert not ok((2, 2, 28, 28), (32, 2, 3, 3))                # Cin kh kw = 18 > 16
    assert not ok((2, 1, 28, 28), (33, 1, 3, 3))                # Cout 33
    assert not ok((2, 1, 6, 6), (4, 1, 3, 3))                   # 36 outputs per plane (not a multiple of 8)
    assert not ok((2, 1, 48, 48), (4, 1, 3, 3))                 # a padded plane of 2500 floats
    assert not ok((0, 1, 28, 28), (32, 1, 3, 3))                # no samples
    L = nnh.lib()
    assert L.nnh_conv2d_packed_supported(1, 1, 28, 28, 32, 3, 3, 1, 1, 0) == 1


def test_empty_products_touch_nothing_and_need_no_device():
    """m == 0 or n == 0 returns before any device work (gemm.cpp:344); null pointers are then fine."""
    assert _sgemm(0, 0, 0, 5, 4, None, 4, None, 5, None, 5, 0, None) == nnh.OK
    assert _sgemm(0, 0, 3, 0, 4, None, 4, None, 1, None, 1, 1, None) == nnh.OK


def test_matmul_shapes_follow_the_reference():
    """tests/test_tensor.cpp:385-392 and 444-450: result shapes and TensorShapeError cases."""
    assert nnh.matmul_shape((2, 3), (3, 2)) == (2, 2)
    assert nnh.matmul_shape((0, 3), (3, 2)) == (0, 2)
    assert nnh.matmul_shape((2, 0), (0, 3)) == (2, 3)
    assert nnh.matmul_shape((2, 3), (3, 0)) == (2, 0)
    assert nnh.matmul_shape((3, 4), (3, 5), True, False) == (4, 5)
    assert nnh.matmul_shape((4, 7, 33), (33, 5)) == (4, 7, 5)          # fold path
    assert nnh.matmul_shape((1, 7, 33), (4, 33, 5)) == (4, 7, 5)       # broadcast
    assert nnh.matmul_shape((2, 1, 9, 7), (1, 3, 6, 9), True, True) == (2, 3, 7, 6)
    for a, b, ta, tb in (((3, 4), (3, 5), 0, 0), ((3, 4), (3, 5), 0, 1), ((3,), (3, 5), 0, 0),
                         ((2, 3, 4), (3, 4, 5), 0, 0), ((2, 3), (4, 2), 0, 0)):
        with pytest.raises(nnh.ShapeError):
            nnh.matmul_shape(a, b, ta, tb)


def test_matmul_shapes_and_errors_match_nncpp(ref):
    """Result shapes and shape errors agree with nn::matmul itself over random shape combinations."""
    import numpy as np
    rng = np.random.default_rng(11)
    for _ in range(300):
        an, bn = int(rng.integers(1, 5)), int(rng.integers(1, 5))
        dims = lambda n: tuple(int(d) for d in rng.choice([1, 2, 3], n))
        a_shape, b_shape = dims(an), dims(bn)
        ta, tb = bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
        rc, out = ref.matmul(np.ones(a_shape, np.float32), np.ones(b_shape, np.float32), ta, tb)
        try:
            got = nnh.matmul_shape(a_shape, b_shape, ta, tb)
            assert rc == 0 and out.shape == got, (a_shape, b_shape, ta, tb)
        except nnh.ShapeError:
            assert rc == 2, (a_shape, b_shape, ta, tb)


def test_workspace_queries_on_the_host():
    """The *_workspace_size queries need no device: nn-cpp's depth cut (gemm.cpp:453-458) decides the GEMM's partials,
    128-deep pieces of m n floats each where there are more than 16 pieces (up to 16, one launch adds them in LDS),
    and the multi-step ops take the largest of their pieces. The queries answer for both numerics modes: the
    split-depth mode's cuts have at most 16 pieces, so they add nothing here."""
    import nnh
    assert nnh.workspace_size("sgemm", 64, 64, 4096, 1) == 32 * 64 * 64 * 4
    assert nnh.workspace_size("sgemm", 40, 48, 2200, 3) == 18 * 40 * 48 * 4 * 3
    assert nnh.workspace_size("sgemm", 512, 512, 512, 1) == 0          # m n > 2^16: no cut (split mode: 16 pieces)
    assert nnh.workspace_size("sgemm", 16, 16, 2048, 1) == 0           # m n k < 2^20: no cut
    assert nnh.workspace_size("sgemm", 256, 10, 1024, 1) == 0          # 8 pieces: one launch, no partials
    assert nnh.workspace_size("sgemm", 40, 48, 2048, 64) == 0          # 16 pieces: one launch
    assert nnh.workspace_size("matmul", [2, 40, 2200], 3, [2200, 48], 2, 0, 0) == 18 * 80 * 48 * 4  # folded: 80 x 48
    assert nnh.workspace_size("matmul", [3, 40, 2200], 3, [3, 2200, 48], 3, 0, 0) == 18 * 40 * 48 * 4 * 3
    assert nnh.workspace_size("linear_forward", 40, 2200, 48) == 18 * 40 * 48 * 4
    assert nnh.workspace_size("linear_forward", 40, 1100, 48) == 0     # 9 pieces: one launch
    # linear backward: dW = G^T X is 48 x 1100 x 40 (no cut), dX = G W is 40 x 1100 x 48 (no cut); a 3-D input's
    # bias gradient takes two buffers of lead[1] * n floats
    assert nnh.workspace_size("linear_backward", [40], 1, 1100, 48, 1, 1, 1) == 0
    assert nnh.workspace_size("linear_backward", [3, 5], 2, 20, 7, 0, 0, 1) == 2 * 256
    # conv2d backward at config 3's conv2 (batch 128, 32 -> 64 on 14 x 14): masked gradient, per-sample db and dW
    # (dx keeps dcol on chip for 196 positions)
    N, Cout, hw, K = 128, 64, 196, 288
    r = lambda b: (b + 255) // 256 * 256
    assert nnh.workspace_size("conv2d_backward", N, 32, 14, 14, Cout, 3, 3, 1, 1, 1, 1, 1, 1) == \
        r(N * Cout * hw * 4) + r(N * Cout * 4) + r(N * Cout * K * 4)
    assert nnh.workspace_size("conv2d_forward", N, 1, 28, 28, 32, 3, 3, 1, 1) == 0  # direct kernel
    # attention backward at config 4: dS, one float per score
    assert nnh.workspace_size("attention_backward", 32, 256, 256, 512, 8) == 32 * 8 * 256 * 256 * 4
    with pytest.raises(nnh.ShapeError):
        nnh.workspace_size("attention_backward", 2, 4, 4, 10, 3)  # heads must divide D

"""nn::matmul / nn::matmul_bt backward on the GPU (nnh_matmul_backward) against nn-cpp's own backward rules
(src/autograd/ops.cpp:683-712, 747-773, run on its compiled sources), bit for bit: the folded path (b a 2-D matrix:
sgemm straight into the gradient with accumulate = !first), the batched path (a Tensor matmul reduced over
broadcast axes by sum_to_shape, then stored as term + 0.0f or added), a depth-cut product, fresh and accumulated
gradients, and one tensor used as both operands."""
import numpy as np
import pytest

from helpers import assert_same
from nnh import synth

pytestmark = pytest.mark.gpu

# (a shape, b shape, matmul_bt)
CASES = [
    ((7, 33), (33, 5), False),                 # 2-D: folded
    ((4, 7, 33), (33, 5), False),              # folded: a's leading axes into M
    ((2, 3, 7, 33), (5, 33), True),            # matmul_bt folded
    ((2048, 40), (40, 48), False),             # dB = A^T G takes nn-cpp's depth cut (40 x 48 x 2048)
    ((3, 7, 33), (3, 33, 5), False),           # batched, same batch: no reduction
    ((1, 7, 33), (4, 33, 5), False),           # a broadcast over the batch: grad_a summed over axis 0, kept as 1
    ((7, 33), (4, 33, 5), False),              # a 2-D against a batched b: grad_a summed over the extra axis
    ((2, 1, 7, 9), (1, 3, 9, 6), False),       # two broadcast axes, one on each side
    ((2, 3, 16, 8), (2, 3, 16, 8), True),      # composed attention's scores: q_h k_h^T per (sample, head)
    ((2, 3, 16, 16), (2, 3, 16, 8), False),    # composed attention's output: P v_h
    ((3, 5, 600), (3, 600, 40), False),        # batched with a depth cut in dA? (5 x 600 x 40: no); dB 600x40x5
    ((16, 4, 64, 16), (16, 4, 64, 16), True),  # transformer_tiny's scores: both gradients in one launch
    ((16, 4, 64, 64), (16, 4, 64, 16), False), # and its P v_h
]


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("case", CASES)
def test_matmul_backward_matches_nncpp(gpu, ref, case):
    """Fresh gradients (where both run on the chain kernel, in one launch), then accumulated ones, against nn-cpp's
    own backward rule."""
    import nnh
    import torch
    ash, bsh, bt = case
    a, b = synth.uniform_operands(hash(case) % 1000 + 7, [ash, bsh])
    out_shape = nnh.matmul_shape(ash, bsh, False, bt)
    g = synth.normal(11, out_shape)
    da_a, db_a = dev(a), dev(b)
    for repeats in (1, 2):
        da = torch.full(ash, float("nan"), device="cuda")
        db = torch.full(bsh, float("nan"), device="cuda")
        for r in range(repeats):
            nnh.matmul_backward(dev(g), da_a, db_a, bt, da, r == 0, db, r == 0)
        torch.cuda.synchronize()
        want_a, want_b = ref.matmul_backward(a, b, bt, g, repeats)
        assert_same(host(da), want_a, ("da", case, repeats))
        assert_same(host(db), want_b, ("db", case, repeats))


@pytest.mark.parametrize("bt", [False, True])
def test_matmul_backward_one_tensor_both_operands(gpu, ref, bt):
    """matmul(x, x): the reference writes dA first (fresh) and then adds dB into the same gradient."""
    import nnh
    import torch
    x = synth.mt19937_uniform(5, 24 * 24).reshape(24, 24)
    g = synth.normal(12, (24, 24))
    dx = torch.full((24, 24), float("nan"), device="cuda")
    xd = dev(x)
    nnh.matmul_backward(dev(g), xd, xd, bt, dx, True, dx, False)
    torch.cuda.synchronize()
    want, _ = ref.matmul_backward(x, None, bt, g, 1)
    assert_same(host(dx), want, ("one tensor", bt))


def test_matmul_backward_shape_errors(gpu):
    import ctypes as C

    import nnh
    sh = lambda s: (C.c_size_t * len(s))(*s)
    rc = nnh.lib().nnh_matmul_backward(None, None, sh((4, 5)), 2, None, sh((6, 3)), 2, 0, None, 1, None, 1, None)
    assert rc == nnh.ERR_SHAPE

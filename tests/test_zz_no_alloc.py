"""nnh_sgemm_noalloc (include/nnh_noalloc.h): nnh_sgemm with its depth-cut partials in a static device array,
for callers that cannot allocate. Checked through the C ABI against nnh_sgemm, bit for bit, on two calls in a row
(the second smaller, so it runs over what the first left in the shared array), and against the oracle."""
import ctypes as C

import numpy as np
import pytest

from helpers import Problem, assert_same, oracle_sgemm

pytestmark = pytest.mark.gpu


def _run(fn, p, acc):
    import torch

    import nnh
    dev = torch.device("cuda:0")
    a, b = torch.from_numpy(p.a).to(dev), torch.from_numpy(p.b).to(dev)
    c = torch.from_numpy(np.array(p.c, copy=True)).to(dev)
    rc = fn(p.ta, p.tb, p.m, p.n, p.k, nnh._ptr(a), p.lda, nnh._ptr(b), p.ldb, nnh._ptr(c), p.ldc, int(acc),
            nnh._stream(None))
    nnh.check(rc)
    torch.cuda.synchronize()
    return c.cpu().numpy()


# (ta, tb, m, n, k): the first two take nn-cpp's depth cut (m n <= 2^16, k >= 512, m n k >= 2^20) into more than 16
# pieces, so their pieces write partial sums to the scratch; the second is smaller than the first; the third is
# cut into 9 pieces, added in one launch without scratch; the last has no cut
CASES = [(0, 0, 64, 64, 4096), (1, 0, 40, 48, 2200), (0, 1, 40, 48, 1100), (0, 1, 33, 70, 300)]


def test_noalloc_matches_sgemm_on_successive_calls(gpu, oracle):
    import nnh
    L = nnh.lib()
    assert L.nnh_sgemm_noalloc_max_workspace() == 16 << 20
    for acc in (False, True):
        for i, (ta, tb, m, n, k) in enumerate(CASES):
            p = Problem(ta, tb, m, n, k, pad=3, seed=900 + i)
            print(f"noalloc case {(ta, tb, m, n, k)} acc={acc}", flush=True)
            got = _run(L.nnh_sgemm_noalloc, p, acc)
            want = _run(L.nnh_sgemm, p, acc)
            assert_same(got, want, ("noalloc vs nnh_sgemm", ta, tb, m, n, k, acc))
            assert_same(got, oracle_sgemm(oracle, p, acc), ("noalloc vs oracle", ta, tb, m, n, k, acc))


def test_noalloc_rejects_partials_beyond_its_array(gpu):
    """256 x 256 x 8320 needs 65 pieces of 65536 floats (17 MB) of partials: refused before any launch, C intact."""
    import torch

    import nnh
    L = nnh.lib()
    m = n = 256
    k = 8320
    a = torch.zeros((m, k), device="cuda")
    b = torch.zeros((k, n), device="cuda")
    c = torch.full((m, n), 7.0, device="cuda")
    rc = L.nnh_sgemm_noalloc(0, 0, m, n, k, nnh._ptr(a), k, nnh._ptr(b), n, nnh._ptr(c), n, 0, nnh._stream(None))
    assert rc == nnh.ERR_INVALID
    assert b"static scratch" in L.nnh_last_error()
    torch.cuda.synchronize()
    assert bool((c == 7.0).all())

"""Shared fixtures. GPU tests (marker `gpu`) call the product through its C ABI (nn-cpp_amd/lib/libnnh.so)
and check it against the oracle (oracle/), which restates nn-cpp bit for bit and is pinned to nn-cpp's
own compiled sources and golden vectors by the CPU tests."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "nn-cpp_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))

SENTINEL = np.float32(1e30)  # tests/test_kernels.cpp:22 kSentinel


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libnnh.so")


@pytest.fixture(scope="session")
def oracle():
    from pyoracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from pyoracle import Reference, reference_available
    if not reference_available():
        pytest.skip("oracle/_ref/libnnref.so not built (needs /root/reference at build time)")
    return Reference()


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    import nnh
    nnh.lib()  # fails loudly when the HIP library is missing
    return torch.device("cuda:0")

"""Host sanitizers over libnnh's host code, on the CPU (no GPU needed).

* ``abi_sanitize``: every include/nnh.h entry point called with valid and invalid arguments against the C-ABI
  translation units built with -fsanitize=address,undefined. Valid calls reach the HIP runtime and come back
  NNH_ERR_HIP (no device here); invalid ones are refused with their code first. Sizes past every limit (2^31
  dimensions, leading dimensions and strides near 2^63, shape products past 64 bits) check that the validation's
  own arithmetic stays defined: an overflow there is an UndefinedBehaviorSanitizer report and fails the test.
* ``workspace_asan`` / ``workspace_tsan``: the per-(device, stream) scratch table behind every call that needs
  device scratch (nn-cpp_amd/src/workspace_table.hpp), on a host stand-in for the runtime, from eight threads at
  once with a caller-registered buffer toggled meanwhile and allocation failures injected, under
  -fsanitize=address,undefined and under -fsanitize=thread.

The programs and their build are tests/cpp/{abi_sanitize,workspace_sanitize}.cpp and tests/cpp/Makefile's
``sanitize`` target.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP = os.path.join(ROOT, "tests", "cpp")
SAN = os.path.join(CPP, "lib", "san")


@pytest.fixture(scope="module")
def built():
    r = subprocess.run(["make", "-j8", "-C", CPP, "sanitize"], capture_output=True, text=True)
    if r.returncode != 0:
        pytest.fail("sanitizer build failed:\n" + r.stdout[-3000:] + r.stderr[-3000:])
    return SAN


def _run(path, *args, timeout=300):
    env = dict(os.environ)
    env["ASAN_OPTIONS"] = "abort_on_error=0:halt_on_error=1:detect_leaks=1"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    env["TSAN_OPTIONS"] = "halt_on_error=1:second_deadlock_stack=1"
    return subprocess.run([path, *args], capture_output=True, text=True, timeout=timeout, env=env)


def _check(r, marker):
    out = r.stdout + r.stderr
    assert "Sanitizer" not in out, out[-4000:]
    assert r.returncode == 0, out[-4000:]
    assert marker in r.stdout, out[-4000:]


def test_abi_validation_under_address_and_ub_sanitizers(built):
    r = _run(os.path.join(built, "abi_sanitize"))
    if r.returncode == 77:
        pytest.skip(r.stdout.strip())
    _check(r, "every code as expected")


def test_workspace_table_under_address_and_ub_sanitizers(built):
    _check(_run(os.path.join(built, "workspace_asan"), "4000"), "all checks passed")


def test_workspace_table_under_thread_sanitizer(built):
    _check(_run(os.path.join(built, "workspace_tsan"), "4000"), "all checks passed")

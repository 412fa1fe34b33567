"""The CPU oracle and the C-ABI library's host code under AddressSanitizer and
UndefinedBehaviorSanitizer (tests/sanitize/Makefile): the oracle over
edge-case rows in exactly sized buffers, and every entry point's argument
checks, including sizes at the edge of int64 that must be rejected before
any size arithmetic overflows.  CPU only: no call reaches a GPU."""

import os
import shutil
import subprocess

import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sanitize")

pytestmark = pytest.mark.skipif(not os.path.exists(os.path.join(HERE, "Makefile")),
                                reason="the sanitizer checkers are not in this tree")


def _make(target: str) -> str:
    r = subprocess.run(["make", "-s", "-j8", "-C", HERE, target], capture_output=True, text=True,
                       timeout=1200)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-6000:]
    assert "runtime error" not in out and "ERROR: AddressSanitizer" not in out, out[-6000:]
    return out


def test_oracle_under_asan_and_ubsan():
    if not shutil.which("gcc"):
        pytest.skip("gcc not found")
    out = _make("run-oracle")
    assert "oracle sanitizer checks:" in out and ", 0 failed" in out


def test_capi_argument_checks_under_asan_and_ubsan():
    if not os.path.exists(os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")):
        pytest.skip("hipcc not found")
    out = _make("run-capi")
    assert "C-ABI sanitizer checks:" in out and ", 0 failed" in out

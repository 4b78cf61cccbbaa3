"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer
(leak checks on), with injected host allocation failures: tests/native/host_checks.cpp
drives the layout-only state, snapshot part lists, the saved-sequence pool in
bookkeeping mode and the host-side validation of the device entry points. No
GPU is used; the device code in the binary is never launched."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native")
CLANG = "/opt/rocm/llvm/bin/clang++"


@pytest.mark.skipif(not os.path.exists(CLANG) or shutil.which("make") is None, reason="needs the ROCm clang")
def test_host_code_under_sanitizers():
    jobs = str(min(8, os.cpu_count() or 1))
    b = subprocess.run(["make", "-s", "-j", jobs, "-C", HERE], capture_output=True, text=True, timeout=900)
    assert b.returncode == 0, b.stdout[-3000:] + b.stderr[-3000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([os.path.join(HERE, "_build", "host_checks")], capture_output=True, text=True, timeout=300,
                       env=env)
    assert r.returncode == 0 and "host checks ok" in r.stdout, r.stdout[-3000:] + r.stderr[-6000:]

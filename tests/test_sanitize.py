"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (gcc, no GPU
code): the product's host layer (ops.cpp: guards, gfx950 tile selection over
extreme shapes, the C-ABI) with the HIP launch layer replaced by checking
stubs, the product's host headers, and the CPU oracle on edge inputs
(tests/native/sanitize_main.cpp).  Any sanitizer report aborts the driver."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
NATIVE = os.path.join(HERE, "native")


@pytest.mark.skipif(shutil.which("gcc") is None or shutil.which("g++") is None,
                    reason="gcc/g++ not present")
def test_host_code_under_asan_and_ubsan():
    subprocess.run(["make", "-s", "-C", NATIVE, "sanitize"], check=True, timeout=600)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1", OMP_NUM_THREADS="4")
    r = subprocess.run([os.path.join(NATIVE, "_san", "sanitize_check")], capture_output=True,
                       text=True, timeout=600, env=env)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "all checks passed" in r.stdout
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr

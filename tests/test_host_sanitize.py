"""Sanitizer builds on the CPU (no GPU): the oracle C under ASan + UBSan
(`make -C oracle sanitize`, every exported function on exact-size buffers),
and the HIP library's host code -- argument checks, error state, planners --
under ASan + UBSan (build.build_host_sanitized), driven by the CPU tests of
the C ABI in a child process with clang's ASan runtime preloaded."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_oracle_under_asan_and_ubsan():
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    res = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "sanitize"], capture_output=True,
                         text=True, timeout=600)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-4000:]
    assert "sanitize_check: ok" in res.stdout
    # a write one word past a buffer, planted in the oracle driver, is reported
    planted = subprocess.run([os.path.join(ROOT, "oracle", "_build", "sanitize_check"), "planted"],
                             capture_output=True, text=True, timeout=60)
    assert planted.returncode != 0 and "heap-buffer-overflow" in planted.stderr, planted.stderr[-2000:]


def test_host_code_under_asan_and_ubsan():
    from eredu_amd import build as B

    if not os.path.exists(B.HIPCC):
        pytest.skip("hipcc not available")
    lib = B.build_host_sanitized()
    runtime = B.sanitizer_runtime()
    assert os.path.exists(runtime), runtime
    env = dict(os.environ, LD_PRELOAD=runtime, EREDU_AMD_LIB=lib,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:halt_on_error=1",  # the interpreter itself leaks
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    tests = [os.path.join(ROOT, "tests", f) for f in ("test_boundary.py", "test_dispatch.py", "test_checkpoint.py")]
    res = subprocess.run([sys.executable, "-m", "pytest", "-q", "-m", "not gpu", "-p", "no:cacheprovider", *tests],
                         cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    assert res.returncode == 0, res.stdout[-4000:] + res.stderr[-4000:]
    assert "ERROR: AddressSanitizer" not in res.stderr and "runtime error" not in res.stderr

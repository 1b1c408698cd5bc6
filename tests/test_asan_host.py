"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU: tests/asan/Makefile
builds every source with the sanitizers on the host side (device code as usual) and links tests/asan/abi_host.c,
which drives config validation, argument checks, forged and NULL handles and the no-device error of the C ABI.
A memory or undefined-behaviour error aborts the driver; a wrong status makes it exit non-zero."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
OUT = os.path.join(ROOT, "_build", "asan")

pytestmark = pytest.mark.skipif(not os.path.exists("/opt/rocm/bin/hipcc") or shutil.which("make") is None,
                                reason="hipcc or make is missing")


def test_host_paths_clean_under_asan_and_ubsan():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("the driver checks the no-device paths")
    b = subprocess.run(["make", "-s", "-j8", "-C", os.path.join(ROOT, "tests", "asan"), "OUT=" + OUT],
                       capture_output=True, text=True, timeout=600)
    assert b.returncode == 0, b.stdout + b.stderr
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="halt_on_error=1")
    r = subprocess.run([os.path.join(OUT, "abi_host")], capture_output=True, text=True, timeout=120, env=env,
                       cwd="/tmp")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "abi_host: 0 failures" in r.stdout

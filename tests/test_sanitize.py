"""The library's host code under sanitizers: tests/sanitize/host_stress.cpp
(8 threads sharing one allocator and planner; two processes and two
receiving threads on one channel, host payloads) built from the library's
sources with the host pass under AddressSanitizer + UndefinedBehaviorSanitizer
and under ThreadSanitizer (tests/sanitize/Makefile).  CPU only: the driver
never touches a GPU, and the device code is built but not run."""
import os
import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent / "sanitize"
HIPCC = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "bin" / "hipcc"


@pytest.fixture(scope="module")
def built():
    if not HIPCC.exists() or shutil.which("make") is None:
        pytest.skip("hipcc or make not available")
    r = subprocess.run(["make", "-C", str(HERE), "all"], capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    return HERE / "_build"


@pytest.mark.parametrize("variant,env", [
    ("asan", {"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0", "UBSAN_OPTIONS": "print_stacktrace=1"}),
    ("tsan", {"TSAN_OPTIONS": "halt_on_error=1"}),
])
def test_host_stress_is_clean(built, variant, env):
    r = subprocess.run([str(built / f"host_stress_{variant}")], capture_output=True, text=True, timeout=600,
                       env=dict(os.environ, **env))
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "host stress ok" in out
    for marker in ("AddressSanitizer", "LeakSanitizer", "runtime error:", "ThreadSanitizer"):
        assert marker not in out, out[-4000:]

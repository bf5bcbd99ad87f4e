"""The library used from C alone: tests/c_abi/pace_kv_check (built by
paceserve_amd.build next to its source) packs and unpacks pages and sends
them through a cross-process channel, through include/pace_kv.h with the HIP
runtime, and checks every byte on the host."""
import subprocess

import pytest

from paceserve_amd.build import C_CHECK_BIN

pytestmark = pytest.mark.gpu


def test_c_program_packs_and_unpacks_through_the_header(gpu):
    if not C_CHECK_BIN.exists():
        pytest.fail(f"{C_CHECK_BIN} is not built (run python -m paceserve_amd.build)")
    r = subprocess.run([str(C_CHECK_BIN)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "C ABI check passed" in r.stdout and "channel" in r.stdout

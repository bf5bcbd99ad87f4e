"""The library used from C alone: tests/c_abi/pace_kv_check (built by
paceserve_amd.build next to its source) packs and unpacks pages, sends them
through a cross-process channel, stages them through pinned host memory,
swaps them out and in, appends tokens, moves pages and packs them without
allocating, through include/pace_kv.h with the HIP runtime, and checks every
byte on the host."""
import json
import subprocess

import pytest

from paceserve_amd.build import C_CHECK_BIN, C_LATENCY_BIN

pytestmark = pytest.mark.gpu


def test_c_program_packs_and_unpacks_through_the_header(gpu):
    if not C_CHECK_BIN.exists():
        pytest.fail(f"{C_CHECK_BIN} is not built (run python -m paceserve_amd.build)")
    r = subprocess.run([str(C_CHECK_BIN)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "C ABI check passed" in r.stdout
    for leg in ("channel", "staged", "swapped", "appended", "moved", "without allocating"):
        assert leg in r.stdout, leg


def test_c_promote_latency_program_moves_the_right_bytes(gpu):
    """tests/c_abi/pace_kv_promote_latency (the bench's C-caller promote
    latency) on a small request: 4 layers, 12 of 64 pages of 4 KiB, both
    modes; it checks every moved page of three layers and of the buffer."""
    if not C_LATENCY_BIN.exists():
        pytest.fail(f"{C_LATENCY_BIN} is not built (run python -m paceserve_amd.build)")
    r = subprocess.run([str(C_LATENCY_BIN), "4", "64", "12", "4096", "5", "1"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert res["verified"] is True and res["n_pages"] == 12
    assert res["buffer"]["p50_us"] > 0 and res["fused"]["p50_us"] > 0

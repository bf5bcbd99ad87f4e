import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libpace_kv.so")


def pytest_sessionstart(session):
    """Builds libpace_kv.so and the C checker when a checkout has neither
    (they are build outputs, not sources); a tree that has them is used as
    it is."""
    from paceserve_amd import build

    if not build.LIB_PATH.exists():
        build.build_library()
    if not build.C_CHECK_BIN.exists():
        build.build_c_check()


def gpu_available() -> bool:
    if not os.path.exists("/dev/kfd"):
        return False
    import torch
    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def gpu():
    """Skips unless a GPU is present; fails loudly if the HIP library is missing."""
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    from paceserve_amd import _native
    _native.load()
    return torch.device("cuda", 0)

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "needle-rs_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (run on the MI355X box)")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def nh():
    """The product package, initialised on cuda:0 (GPU tests only)."""
    if not _gpu_available():
        pytest.fail("GPU test collected without a visible GPU")
    import needle_hip

    needle_hip.init(0)
    return needle_hip


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle

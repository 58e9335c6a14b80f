import sys
from pathlib import Path

import pytest

sys.path.insert(0, str(Path(__file__).resolve().parent))
sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def oracle():
    from helpers import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def zest_gpu():
    """The package with its library loaded and device 0 initialised; the GPU
    tests must run through it (no fallback)."""
    import torch
    from helpers import load_pkg
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a GPU")
    z = load_pkg()
    z.init(0)
    return z

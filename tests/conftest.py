import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu on the GPU box")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def hip():
    """The HIP kernel library on a GPU box; GPU tests fail loudly if it is missing."""
    import torch
    import tensorvia_amd as tv
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    tv.lib()
    return tv

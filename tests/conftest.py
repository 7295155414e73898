import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """Skip unless a GPU is present; fail loudly if it is but the HIP library is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from navi_amd import _native  # raises ImportError (test error) if unbuilt

    return _native

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def pytest_collection_modifyitems(config, items):
    """GPU tests fail loudly (not skip) when a GPU is expected; without one they are deselected by -m "not gpu"."""
    return None


@pytest.fixture(scope="session")
def lib():
    """The built C-ABI library (HIP path). Raises if it was not built: the product has no fallback."""
    from heimdall_amd import _lib
    return _lib.load()


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    return torch.device("cuda:0")


os.environ.setdefault("PYTHONHASHSEED", "0")

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

_MARGINS = []


@pytest.fixture
def margin(request):
    """margin(name, err, tol): assert a parity error is below its tolerance and keep the measurement, so every
    full-size check's margin appears in the run's log (the table printed at the end of the session, also under -q,
    and the test's user_properties for junit-xml)."""
    def rec(name, err, tol):
        err, tol = float(err), float(tol)
        _MARGINS.append((request.node.name, name, err, tol))
        request.node.user_properties.append((name, err))
        assert err < tol, f"{name}: {err:.3e} is not below {tol:.1e}"
    return rec


def pytest_terminal_summary(terminalreporter):
    if not _MARGINS:
        return
    tr = terminalreporter
    tr.section("parity margins: relative L2 error against the oracle / tolerance")
    for test, name, err, tol in _MARGINS:
        tr.write_line(f"{test} | {name}: {err:.3e} / {tol:.0e} = {err / tol:.3f} of the tolerance")

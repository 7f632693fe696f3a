"""CPU checks of the C-ABI boundary: the library loads and exports every symbol declared in include/bifrost.h,
argument errors come back as status codes without a GPU, and the ctypes signatures cover the header."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "bifrost.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bf_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def cpu_lib():
    from heimdall_amd import _lib
    if not _lib.LIB_PATH.exists():                 # the build check builds it; a bare test run builds it here
        from heimdall_amd.build import build_library
        build_library()
    return _lib.load()


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "bf_gdn_fwd" in syms and "bf_gdn_workspace_size" in syms and len(syms) >= 4


def test_library_exports_every_declared_symbol(cpu_lib):
    missing = [s for s in declared_symbols() if not hasattr(cpu_lib, s)]
    assert not missing, missing


def test_ctypes_signatures_cover_header():
    from heimdall_amd import _lib
    assert sorted(_lib.SIGNATURES) == declared_symbols()


def declared_arity():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for name, args in re.findall(r"\b(bf_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        args = args.strip()
        out[name] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def test_ctypes_arity_matches_header():
    from heimdall_amd import _lib
    ar = declared_arity()
    assert sorted(ar) == declared_symbols()
    for name, (_, argtypes) in _lib.SIGNATURES.items():
        assert len(argtypes) == ar[name], (name, len(argtypes), ar[name])


def test_status_codes_without_gpu(cpu_lib):
    assert cpu_lib.bf_version() >= 100
    assert cpu_lib.bf_status_string(0) == b"ok"
    n = ctypes.c_size_t(0)
    assert cpu_lib.bf_gdn_workspace_size(4096, 1, 4, 1, 256, 1, 0, ctypes.byref(n)) == 0 and n.value > 0
    assert cpu_lib.bf_gdn_workspace_size(4096, 1, 4, 1, 96, 1, 0, ctypes.byref(n)) == -2      # unsupported D
    assert cpu_lib.bf_gdn_workspace_size(4096, 0, 4, 1, 256, 1, 0, ctypes.byref(n)) == -1     # no sequences
    assert cpu_lib.bf_gdn_workspace_size(4096, 1, 4, 1, 256, 1, -1, ctypes.byref(n)) == -1    # bad segment length
    # argument errors are reported before anything is launched (null workspace)
    st = cpu_lib.bf_gdn_fwd(1, 1, 1, 1, 1, None, 1, 64, 4, 1, 256, 1, 1.0, None, 1, 0, None, 0, None, 0, 7, None)
    assert st == -3
    st = cpu_lib.bf_gdn_fwd(1, 1, 1, 1, 1, None, 3, 64, 4, 1, 256, 1, 1.0, None, 1, 0, None, 0, None, 0, 7, None)
    assert st == -1                                                                            # 64 % 3 != 0
    st = cpu_lib.bf_gdn_fwd(1, 1, 1, 1, 1, None, 1, 64, 4, 1, 256, 1, 1.0, None, 1, 0, None, 0, None, 0, 16, None)
    assert st == -1                                                                            # unknown phase bit
    st = cpu_lib.bf_gdn_fwd(1, 1, 1, 1, 1, None, 1, 64, 4, 1, 256, 1, 1.0, None, 1, 0, None, 0, None, 0, 0, None)
    assert st == -1                                                                            # no phase


def test_workspace_size_grows_with_tokens(cpu_lib):
    a, b = ctypes.c_size_t(0), ctypes.c_size_t(0)
    cpu_lib.bf_gdn_workspace_size(4096, 1, 4, 1, 256, 1, 0, ctypes.byref(a))
    cpu_lib.bf_gdn_workspace_size(8192, 1, 4, 1, 256, 1, 0, ctypes.byref(b))
    assert b.value > a.value
    # shorter segments need more per-segment summaries
    cpu_lib.bf_gdn_workspace_size(8192, 1, 4, 1, 256, 1, 2, ctypes.byref(a))
    cpu_lib.bf_gdn_workspace_size(8192, 1, 4, 1, 256, 1, 64, ctypes.byref(b))
    assert a.value > b.value


def test_product_has_no_cpu_path():
    """The operators refuse CPU tensors instead of falling back."""
    import torch
    from heimdall_amd import kernels
    from heimdall_amd._lib import BifrostError
    q = torch.zeros(1, 4, 1, 64)
    with pytest.raises(BifrostError):
        kernels.delta_rule(q, q, q, torch.zeros(1, 4, 1), torch.zeros(1, 4, 1))

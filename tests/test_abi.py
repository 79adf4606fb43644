"""C-ABI library (CPU-side checks: no GPU calls): it loads and exports every entry point include/atl_hip.h
declares, and the host-side wrappers reject bad arguments before any launch."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "atl_hip.h").read_text()
    return sorted(set(re.findall(r"\b(atl_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from x_amd.ops import _ext
    if not _ext.LIB_PATH.exists():
        from x_amd.csrc.build import build
        build()
    return ctypes.CDLL(str(_ext.LIB_PATH))


def test_library_exports_every_declared_symbol(lib):
    names = declared_symbols()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_shim_binds_every_declared_symbol():
    from x_amd.ops import _ext
    bound = set(_ext._SIGS) | {"atl_last_error", "atl_abi_version"}
    assert set(declared_symbols()) <= bound


def test_abi_version_and_error_path(lib):
    from x_amd.ops import _ext
    L = _ext.load_library()
    assert L.atl_abi_version() == 1
    # a rejected argument never launches: negative size -> status 1 and a message
    rc = L.atl_splat_bilinear_fwd(None, None, None, -1, 1, 4, 4, None, None)
    assert rc == 1 and b"bad sizes" in L.atl_last_error()
    rc = L.atl_ats_pair_fwd(*([None] * 5), 0, 7, *([None] * 4), 0, None, 16, 3, 4, 1.0, 0.2, 3.0, None, None, None)
    assert rc == 1 and b"ats_pair_fwd" in L.atl_last_error()

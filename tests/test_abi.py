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


def test_workspace_and_trajectory_entries_reject_before_launch(lib):
    """The reference-layout workspace entries and the trajectory origin entries check their arguments and
    workspace on the host and return status 1 with a message, without a launch (no device is touched)."""
    import ctypes
    from x_amd.ops import _ext
    L = _ext.load_library()
    assert L.atl_ats_pair_ws_bytes(-1, 10, 10, 4) == -1
    need = L.atl_ats_pair_ws_bytes(100, 48, 10, 4)
    assert need > 0
    fake = ctypes.c_void_p(256)                    # an aligned, never dereferenced address
    args = (*([None] * 5), 100, 48, *([None] * 4), 10, None, 4, 3, 4, 1.0, 0.2, 3.0)
    rc = L.atl_ats_pair_fwd_ws(*args, None, None, fake, need - 1, None)
    assert rc == 1 and b"workspace" in L.atl_last_error()
    rc = L.atl_ats_pair_bwd_ws(None, *args, 10, None, fake, need - 1, None)
    assert rc == 1 and b"workspace" in L.atl_last_error()
    rc = L.atl_ats_pair_fwd_ws(*(args[:6] + (47,) + args[7:]), None, None, fake, need, None)  # ncell % (GH GW)
    assert rc == 1 and b"bad arguments" in L.atl_last_error()
    rc = L.atl_traj_origin(None, 1, 6, 4, 8, 8, None, None, None, 5, 6, 0.0, 1, 2, None, 0, None, None)
    assert rc == 1 and b"expected 2K" in L.atl_last_error()
    rc = L.atl_traj_origin_bwd(None, 1, 8, 4, 8, 8, None, None, None, 5, 0, 1, None, None, None, None)
    assert rc == 1 and b"traj_origin_bwd" in L.atl_last_error()

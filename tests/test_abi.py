"""CPU checks of the drop-in boundary: libtpmd.so loads and exports every
function include/tpmd.h declares (no GPU calls here)."""
import ctypes

import tpmd


def test_library_exports_header_symbols():
    L = ctypes.CDLL(tpmd.LIB_PATH)
    syms = tpmd.header_symbols()
    assert len(syms) >= 20
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing


def test_abi_version_and_null_safety():
    L = tpmd.lib()
    assert L.tpmd_abi_version() == 1
    assert L.tpmd_last_error(None) == b"no context"
    L.tpmd_destroy(None)


def test_shim_driver_is_built():
    """the tp::motion_dec driver links against the library (usage error, no GPU use)"""
    import os
    import subprocess
    shim = os.path.join(os.path.dirname(tpmd.LIB_PATH), "shim_check")
    p = subprocess.run([shim], capture_output=True, text=True, timeout=60)
    assert p.returncode == 2 and "usage" in p.stderr

"""The C-ABI library loads without a GPU and exports every entry point that
include/pyramidkv_hip.h declares; pure host queries answer correctly.  No
compute call is made here."""
import ctypes

from pyramidkv import _abi as A


def test_library_exports_every_declared_symbol():
    lib = A.lib()
    declared = A.declared_symbols()
    assert len(declared) >= 13
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing


def test_host_queries():
    lib = A.lib()
    assert lib.pkv_abi_version() == 3
    assert lib.pkv_perhead_state_size() == 600
    g = A.make_geometry(30, 12, 128, 1560, 3, 24, 4, 8 * 12 * 37 * 1560)
    assert lib.pkv_cache_update_workspace_size(ctypes.byref(g), 3) > 8 * 36 * 4
    assert lib.pkv_merge_workspace_size(12, 3, 1560, 420) >= 36 * (1560 + 421) * 4


def test_argument_errors_are_reported_without_touching_the_device():
    lib = A.lib()
    rc = lib.pkv_ragged_attn_fwd(None, None)
    assert rc == A.PKV_ERR_INVALID
    assert b"NULL" in lib.pkv_last_error()
    rc = lib.pkv_plan_multi(None, None, None, None, None, 0, None, None, None, None)
    assert rc == A.PKV_ERR_INVALID

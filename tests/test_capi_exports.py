"""The C-ABI library loads and exports every entry point include/*.h
declares (no GPU needed; no compute calls)."""
import ctypes
import glob
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    src = "".join(open(p).read() for p in sorted(glob.glob(os.path.join(ROOT, "include", "*.h"))))
    return sorted(set(re.findall(r"GDN2_API\s+[\w\s\*]*?\b(gdn2_\w+)\s*\(", src)))


def test_header_declares_the_boundary():
    syms = declared_symbols()
    for s in ("gdn2_recurrent_step_f32", "gdn2_recurrent_fwd_f32", "gdn2_chunk_fwd_f32",
              "gdn2_chunk_workspace_bytes", "gdn2_decode_fused_f32", "gdn2_hip_available", "gdn2_last_error",
              "gdn2_config_validate", "gdn2_layer_create", "gdn2_layer_forward_f32", "gdn2_layer_forward_train_f32",
              "gdn2_state_create"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    from gdn2_amd import _capi

    lib = ctypes.CDLL(_capi.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    assert set(_capi.EXPORTS) == set(declared_symbols())


def test_library_has_no_oracle_dependency():
    """The product library never links the oracle."""
    from gdn2_amd import _capi

    data = open(_capi.LIB_PATH, "rb").read()
    assert b"gdn2o_" not in data and b"libgdn2_oracle" not in data

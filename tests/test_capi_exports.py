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


def _chunk_ws(B, HV, T, K, V):
    from gdn2_amd import _capi

    lib = ctypes.CDLL(_capi.LIB_PATH)
    lib.gdn2_chunk_workspace_bytes.restype = ctypes.c_size_t
    lib.gdn2_chunk_workspace_bytes.argtypes = [ctypes.POINTER(_capi.ChunkArgs)]
    a = _capi.ChunkArgs()
    a.batch, a.num_heads, a.num_v_heads, a.seq_len, a.head_dim, a.head_v_dim = B, HV, HV, T, K, V
    a.chunk_size = 64
    return lib.gdn2_chunk_workspace_bytes(ctypes.byref(a))


def _per_chunk_ws(B, HV, T, K, V):
    al = lambda x: (x + 255) // 256 * 256
    n = B * HV * ((T + 63) // 64)
    return sum(al(4 * n * e) for e in (64 * K, 64 * K, 64 * V, 64 * 64, 64 * K, K))


def test_chunk_workspace_sizes():
    """Host-only sizing: the per-chunk buffers, plus the segment buffers
    (transitions and entering states) only for few long sequences; shapes
    outside the kernels' instances size without faulting."""
    assert _chunk_ws(8, 16, 4096, 128, 128) == _per_chunk_ws(8, 16, 4096, 128, 128)
    # 1 x 16 heads x 65536 tokens: eight segments of 128 chunks, each with its
    # transition (K x K) and entering state (K x V)
    seg = _chunk_ws(1, 16, 65536, 128, 128) - _per_chunk_ws(1, 16, 65536, 128, 128)
    assert seg == 4 * 16 * (8 * 128 * 128 + 8 * 128 * 128)
    assert _chunk_ws(1, 1, 20, 16, 8) > 0
    assert _chunk_ws(0, 1, 20, 128, 128) == 0

"""ctypes declarations of include/gdn2.h and the loader of libgdn2_amd.so.

The library is built in-tree (burn-gdn2_amd/libgdn2_amd.so) by
burn-gdn2_amd/build.py.  Loading fails loudly when it is missing: there is
no CPU fallback in this package.
"""
from __future__ import annotations

import ctypes
import os

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_ROOT, "libgdn2_amd.so")

GDN2_OK = 0
GDN2_NOT_APPLICABLE = 1
GDN2_EINVAL = 2
GDN2_EHIP = 3

_fp = ctypes.c_void_p
_i64 = ctypes.c_int64
_dbl = ctypes.c_double


class StepArgs(ctypes.Structure):
    _fields_ = [("q", _fp), ("k", _fp), ("g", _fp), ("b", _fp), ("v", _fp), ("w", _fp),
                ("state_in", _fp), ("state_out", _fp), ("out", _fp),
                ("batch", _i64), ("num_heads", _i64), ("num_v_heads", _i64), ("head_dim", _i64),
                ("head_v_dim", _i64),
                ("stride_qk_b", _i64), ("stride_qk_h", _i64), ("stride_vw_b", _i64), ("stride_vw_h", _i64),
                ("stride_o_b", _i64), ("stride_o_h", _i64), ("scale", _dbl)]


class RecurrentArgs(ctypes.Structure):
    _fields_ = [("q", _fp), ("k", _fp), ("g", _fp), ("b", _fp), ("v", _fp), ("w", _fp),
                ("state_in", _fp), ("state_out", _fp), ("out", _fp),
                ("batch", _i64), ("num_heads", _i64), ("num_v_heads", _i64), ("seq_len", _i64),
                ("head_dim", _i64), ("head_v_dim", _i64),
                ("stride_qk_b", _i64), ("stride_qk_h", _i64), ("stride_qk_t", _i64),
                ("stride_vw_b", _i64), ("stride_vw_h", _i64), ("stride_vw_t", _i64),
                ("stride_o_b", _i64), ("stride_o_h", _i64), ("stride_o_t", _i64),
                ("scale", _dbl)]


class ChunkArgs(ctypes.Structure):
    _fields_ = [("q", _fp), ("k", _fp), ("g", _fp), ("b", _fp), ("v", _fp), ("w", _fp),
                ("state", _fp), ("out", _fp),
                ("batch", _i64), ("num_heads", _i64), ("num_v_heads", _i64), ("seq_len", _i64),
                ("head_dim", _i64), ("head_v_dim", _i64),
                ("stride_qk_b", _i64), ("stride_qk_h", _i64), ("stride_qk_t", _i64),
                ("stride_vw_b", _i64), ("stride_vw_h", _i64), ("stride_vw_t", _i64),
                ("stride_o_b", _i64), ("stride_o_h", _i64), ("stride_o_t", _i64),
                ("scale", _dbl), ("chunk_size", _i64),
                ("workspace", _fp), ("workspace_bytes", ctypes.c_size_t)]


class ChunkBwdArgs(ctypes.Structure):
    _fields_ = [("fwd", ChunkArgs), ("d_out", _fp), ("d_state_out", _fp),
                ("dq", _fp), ("dk", _fp), ("dg", _fp), ("db", _fp), ("dv", _fp), ("dw", _fp), ("d_state0", _fp),
                ("workspace", _fp), ("workspace_bytes", ctypes.c_size_t)]


class RecurrentBwdArgs(ctypes.Structure):
    _fields_ = [("fwd", RecurrentArgs), ("d_out", _fp), ("d_state_out", _fp),
                ("dq", _fp), ("dk", _fp), ("dg", _fp), ("db", _fp), ("dv", _fp), ("dw", _fp), ("d_state0", _fp),
                ("workspace", _fp), ("workspace_bytes", ctypes.c_size_t)]


class LayerParams(ctypes.Structure):
    _fields_ = [("q_conv_w", _fp), ("k_conv_w", _fp), ("v_conv_w", _fp), ("a_log", _fp), ("dt_bias", _fp),
                ("decay_factors", _fp), ("o_norm_weight", _fp), ("min_decay", _dbl), ("norm_eps", _dbl),
                ("use_short_conv", ctypes.c_int32), ("allow_neg_eigval", ctypes.c_int32)]


class DecodeArgs(ctypes.Structure):
    _fields_ = [("q_raw", _fp), ("k_raw", _fp), ("f_raw", _fp), ("b_raw", _fp), ("v_raw", _fp),
                ("w_raw", _fp), ("gate", _fp),
                ("conv_q_in", _fp), ("conv_k_in", _fp), ("conv_v_in", _fp),
                ("conv_q_out", _fp), ("conv_k_out", _fp), ("conv_v_out", _fp),
                ("state", _fp), ("out", _fp),
                ("batch", _i64), ("num_heads", _i64), ("num_v_heads", _i64), ("head_dim", _i64),
                ("head_v_dim", _i64), ("scale", _dbl), ("params", ctypes.POINTER(LayerParams))]


class Config(ctypes.Structure):
    """gdn2_config (include/gdn2_layer.h) = Gdn2Config (src/config.rs:23-58)."""
    _fields_ = [("hidden_size", _i64), ("num_heads", _i64), ("head_dim", _i64), ("expand_v", ctypes.c_float),
                ("num_v_heads", _i64), ("use_short_conv", ctypes.c_int32), ("allow_neg_eigval", ctypes.c_int32),
                ("norm_eps", _dbl), ("mode", ctypes.c_int32), ("chunk_size", _i64),
                ("has_min_decay", ctypes.c_int32), ("min_decay", _dbl), ("gva_layout", ctypes.c_int32)]


MODE_FUSED_RECURRENT = 0
MODE_CHUNK = 1
GVA_HEAD_REPEAT = 0
GVA_REFERENCE = 1
STATE_RECURRENT, STATE_CONV_Q, STATE_CONV_K, STATE_CONV_V = 0, 1, 2, 3

# Every symbol include/*.h declares (checked by tests/test_capi_exports.py).
EXPORTS = ("gdn2_last_error", "gdn2_hip_available", "gdn2_recurrent_step_f32", "gdn2_recurrent_fwd_f32",
           "gdn2_chunk_workspace_bytes", "gdn2_chunk_fwd_f32", "gdn2_chunk_intra_f32", "gdn2_chunk_inter_f32",
           "gdn2_chunk_segments", "gdn2_chunk_inter_pass_f32",
           "gdn2_chunk_fwd_states_f32", "gdn2_chunk_noalloc_scratch_bytes", "gdn2_chunk_fwd_noalloc_f32",
           "gdn2_stream_copy_f32", "gdn2_short_conv_f32", "gdn2_l2_normalize_f32", "gdn2_rms_norm_gate_f32",
           "gdn2_chunk_bwd_workspace_bytes", "gdn2_chunk_bwd_f32", "gdn2_chunk_fwd_train_f32",
           "gdn2_chunk_bwd_saved_f32", "gdn2_recurrent_bwd_workspace_bytes",
           "gdn2_recurrent_bwd_f32", "gdn2_decode_fused_f32",
           "gdn2_config_default", "gdn2_config_validate", "gdn2_config_dims", "gdn2_param_count",
           "gdn2_param_name", "gdn2_param_shape", "gdn2_param_init", "gdn2_layer_create", "gdn2_layer_destroy",
           "gdn2_layer_config", "gdn2_layer_set_param", "gdn2_layer_get_param", "gdn2_layer_forward_train_f32",
           "gdn2_layer_forward_f32", "gdn2_layer_project_f32", "gdn2_state_create", "gdn2_state_destroy",
           "gdn2_state_set_zeros", "gdn2_state_clear", "gdn2_state_is_some", "gdn2_state_batch",
           "gdn2_state_numel", "gdn2_state_tensor", "gdn2_state_read", "gdn2_state_write", "gdn2_state_serialize",
           "gdn2_state_deserialize", "gdn2_layer_grads_create", "gdn2_layer_grads_destroy",
           "gdn2_layer_grads_zero", "gdn2_layer_grads_get", "gdn2_layer_backward_f32",
           "gdn2_layer_saved_create", "gdn2_layer_saved_destroy", "gdn2_layer_forward_train_saved_f32")

_lib = None


class Gdn2Error(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"gdn2 status {status}: {msg}")
        self.status = status


def lib():
    """Load libgdn2_amd.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with burn-gdn2_amd/build.py "
                               "(or __graft_entry__.build()); there is no CPU fallback")
        L = ctypes.CDLL(LIB_PATH)
        L.gdn2_last_error.restype = ctypes.c_char_p
        L.gdn2_hip_available.restype = ctypes.c_int
        for name, st in (("gdn2_recurrent_step_f32", StepArgs), ("gdn2_recurrent_fwd_f32", RecurrentArgs),
                         ("gdn2_chunk_fwd_f32", ChunkArgs), ("gdn2_chunk_intra_f32", ChunkArgs),
                         ("gdn2_chunk_fwd_noalloc_f32", ChunkArgs),
                         ("gdn2_chunk_inter_f32", ChunkArgs), ("gdn2_decode_fused_f32", DecodeArgs),
                         ("gdn2_chunk_bwd_f32", ChunkBwdArgs), ("gdn2_chunk_fwd_train_f32", ChunkBwdArgs),
                         ("gdn2_chunk_bwd_saved_f32", ChunkBwdArgs), ("gdn2_recurrent_bwd_f32", RecurrentBwdArgs)):
            fn = getattr(L, name)
            fn.argtypes = [ctypes.POINTER(st), ctypes.c_void_p]
            fn.restype = ctypes.c_int
        L.gdn2_chunk_fwd_states_f32.argtypes = [ctypes.POINTER(ChunkArgs), ctypes.c_void_p, ctypes.c_void_p,
                                                ctypes.c_void_p]
        L.gdn2_chunk_fwd_states_f32.restype = ctypes.c_int
        L.gdn2_chunk_segments.argtypes = [ctypes.POINTER(ChunkArgs)]
        L.gdn2_chunk_segments.restype = _i64
        L.gdn2_chunk_inter_pass_f32.argtypes = [ctypes.POINTER(ChunkArgs), ctypes.c_int, ctypes.c_void_p]
        L.gdn2_chunk_inter_pass_f32.restype = ctypes.c_int
        vp = ctypes.c_void_p
        L.gdn2_short_conv_f32.argtypes = [vp, vp, vp, vp, vp, _i64, _i64, _i64, vp]
        L.gdn2_l2_normalize_f32.argtypes = [vp, vp, _i64, _i64, _dbl, vp]
        L.gdn2_rms_norm_gate_f32.argtypes = [vp, vp, vp, vp, _i64, _i64, _dbl, vp]
        for n in ("gdn2_short_conv_f32", "gdn2_l2_normalize_f32", "gdn2_rms_norm_gate_f32"):
            getattr(L, n).restype = ctypes.c_int
        L.gdn2_stream_copy_f32.argtypes = [ctypes.c_void_p, ctypes.c_void_p, _i64, _i64, ctypes.c_void_p]
        L.gdn2_stream_copy_f32.restype = ctypes.c_int
        L.gdn2_chunk_noalloc_scratch_bytes.argtypes = []
        L.gdn2_chunk_noalloc_scratch_bytes.restype = ctypes.c_size_t
        L.gdn2_chunk_workspace_bytes.argtypes = [ctypes.POINTER(ChunkArgs)]
        L.gdn2_chunk_workspace_bytes.restype = ctypes.c_size_t
        L.gdn2_chunk_bwd_workspace_bytes.argtypes = [ctypes.POINTER(ChunkBwdArgs)]
        L.gdn2_chunk_bwd_workspace_bytes.restype = ctypes.c_size_t
        L.gdn2_recurrent_bwd_workspace_bytes.argtypes = [ctypes.POINTER(RecurrentBwdArgs)]
        L.gdn2_recurrent_bwd_workspace_bytes.restype = ctypes.c_size_t
        _declare_layer(L)
        _lib = L
    return _lib


def _declare_layer(L):
    cfgp, vp, i64, i32, fp = ctypes.POINTER(Config), ctypes.c_void_p, _i64, ctypes.c_int, _fp
    i64p = ctypes.POINTER(_i64)
    sig = {
        "gdn2_config_default": (None, [cfgp]),
        "gdn2_config_validate": (i32, [cfgp]),
        "gdn2_config_dims": (i32, [cfgp, i64p, i64p, i64p, i64p]),
        "gdn2_param_count": (i32, []),
        "gdn2_param_name": (ctypes.c_char_p, [i32]),
        "gdn2_param_shape": (i64, [cfgp, ctypes.c_char_p, i64p, i64p]),
        "gdn2_param_init": (i32, [cfgp, ctypes.c_uint64, ctypes.c_char_p, fp, i64]),
        "gdn2_layer_create": (i32, [cfgp, ctypes.c_uint64, ctypes.POINTER(vp)]),
        "gdn2_layer_destroy": (None, [vp]),
        "gdn2_layer_config": (cfgp, [vp]),
        "gdn2_layer_set_param": (i32, [vp, ctypes.c_char_p, fp, i64]),
        "gdn2_layer_get_param": (i32, [vp, ctypes.c_char_p, fp, i64]),
        "gdn2_layer_forward_train_f32": (i32, [vp, fp, i64, i64, fp, vp]),
        "gdn2_layer_forward_f32": (i32, [vp, fp, i64, i64, vp, fp, vp]),
        "gdn2_layer_project_f32": (i32, [vp, fp, i64, i64, vp, fp, fp, fp, fp, fp, fp, fp, vp]),
        "gdn2_state_create": (i32, [vp, i64, ctypes.POINTER(vp)]),
        "gdn2_state_destroy": (None, [vp]),
        "gdn2_state_set_zeros": (i32, [vp]),
        "gdn2_state_clear": (None, [vp]),
        "gdn2_state_is_some": (i32, [vp]),
        "gdn2_state_batch": (i64, [vp]),
        "gdn2_state_numel": (i64, [vp, i32]),
        "gdn2_state_tensor": (fp, [vp, i32]),
        "gdn2_state_read": (i32, [vp, i32, fp, i64]),
        "gdn2_state_write": (i32, [vp, i32, fp, i64]),
        "gdn2_state_serialize": (i32, [vp, vp, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]),
        "gdn2_state_deserialize": (i32, [vp, vp, ctypes.c_size_t]),
        "gdn2_layer_grads_create": (i32, [vp, ctypes.POINTER(vp)]),
        "gdn2_layer_grads_destroy": (None, [vp]),
        "gdn2_layer_grads_zero": (i32, [vp, vp]),
        "gdn2_layer_grads_get": (i32, [vp, ctypes.c_char_p, fp, i64]),
        "gdn2_layer_backward_f32": (i32, [vp, fp, i64, i64, vp, vp, fp, vp, fp, vp, vp, i32, vp]),
        "gdn2_layer_saved_create": (i32, [vp, i64, i64, ctypes.POINTER(vp)]),
        "gdn2_layer_saved_destroy": (None, [vp]),
        "gdn2_layer_forward_train_saved_f32": (i32, [vp, fp, i64, i64, fp, vp, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def check(status: int, allow_not_applicable=False) -> bool:
    """Raise on error statuses; return False for GDN2_NOT_APPLICABLE when allowed."""
    if status == GDN2_OK:
        return True
    msg = lib().gdn2_last_error().decode(errors="replace")
    if status == GDN2_NOT_APPLICABLE and allow_not_applicable:
        return False
    raise Gdn2Error(status, msg)

"""gdn2_amd: MI355X (gfx950) GDN-2 chunked and recurrent forward, the
chunked backward and the layer's backward.

Python front end of libgdn2_amd.so (C ABI in include/gdn2.h and
include/gdn2_layer.h).  The
operators run hand-written HIP kernels only; when the library is missing
they raise instead of falling back to a CPU path.
"""
from . import _capi
from .layer import GatedDeltaNet2, Gdn2Config, Gdn2Grads, Gdn2Saved, Gdn2State, init_param, init_params, param_names, param_shape
from .ops import (chunk_wy_backward, chunk_wy_forward, chunk_wy_forward_train, chunk_workspace_bytes, decode_fused,
                  fused_recurrent_backward,
                  fused_recurrent_forward, fused_recurrent_gdn2, fused_step, hip_available, l2_normalize,
                  l2_normalize_4d, rms_norm_gate_per_head, short_conv_1d)

__all__ = ["chunk_wy_backward", "chunk_wy_forward", "chunk_wy_forward_train", "chunk_workspace_bytes", "decode_fused", "fused_recurrent_backward", "fused_recurrent_forward",
           "fused_recurrent_gdn2", "fused_step", "hip_available", "l2_normalize", "l2_normalize_4d",
           "rms_norm_gate_per_head", "short_conv_1d", "GatedDeltaNet2", "Gdn2Config", "Gdn2Grads", "Gdn2Saved", "Gdn2State", "init_param", "init_params",
           "param_names", "param_shape", "_capi"]

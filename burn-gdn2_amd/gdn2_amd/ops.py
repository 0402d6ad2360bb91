"""Kernel-level operators on device tensors, named after the reference
functions they replace.  Each builds the C-ABI argument block from torch
tensors (device memory and the current stream only) and calls
libgdn2_amd.so.

  fused_step               src/kernel/fused_recurrent_cube.rs:108-172
  fused_recurrent_forward  src/kernel/fused_recurrent.rs:11-55
  chunk_wy_forward         src/forward.rs:44-278 (+ fused_chunk_forward,
                           src/kernel/chunk_cube.rs:781-952)
  decode_fused             forward() at T == 1, src/module.rs:224-316
  short_conv_1d            src/short_conv.rs:22-65
  l2_normalize(_4d)        src/l2norm.rs:4-16
  rms_norm_gate_per_head   src/module.rs:501-517

Tensor conventions follow the reference: q, k, g, b [B, Hk, T, K];
v, w [B, HV, T, V]; state [B, HV, K, V]; out [B, HV, T, V].  Hk may be
smaller than HV (value head hv reads key head hv // (HV // Hk)); the
reference always materialises Hk == HV.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from . import _capi as C


def _p(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream=None):
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _check_f32_cuda(*ts):
    for t in ts:
        if t is None:
            continue
        if t.dtype != torch.float32 or not t.is_cuda:
            raise TypeError("gdn2_amd operators take float32 device tensors")


def _strides3(t: torch.Tensor):
    if t.stride(3) != 1:
        raise ValueError("the last (channel) dimension must be contiguous")
    return t.stride(0), t.stride(1), t.stride(2)


def _channels_contiguous(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(3) == 1 or t.shape[3] == 1 else t.contiguous()


def _like(t: torch.Tensor, ref: torch.Tensor) -> torch.Tensor:
    """t in ref's shape and layout: a last dim of 1 (per-head scalar g or b,
    src/forward.rs:149,173,180-182) is broadcast over ref's channels, and a
    different layout is copied on the device into ref's."""
    if t.shape == ref.shape and t.stride() == ref.stride():
        return t
    out = torch.empty_strided(ref.shape, ref.stride(), device=ref.device, dtype=torch.float32)
    out.copy_(t.expand(ref.shape))
    return out


def _operands(q, k, v, g, b, w):
    """The kernels read q, k, g, b in one layout and v, w in another, each
    with contiguous channels; other inputs are brought to that form."""
    q, v = _channels_contiguous(q), _channels_contiguous(v)
    return q, _like(k, q), v, _like(g, q), _like(b, q), _like(w, v)


def _reduce_like(grad: torch.Tensor, t: torch.Tensor) -> torch.Tensor:
    """The gradient of an operand broadcast by _like: summed over the
    broadcast channels."""
    return grad.sum(dim=3, keepdim=True) if t.shape[3] == 1 and grad.shape[3] != 1 else grad


def hip_available() -> bool:
    return bool(C.lib().gdn2_hip_available())


def fused_step(q, k, v, g, b, w, state, scale: float, out_state=None) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
    """One decode step (T == 1).  Returns (out [B,HV,1,V], new_state), or
    None when the kernel does not apply (the reference's `None`)."""
    _check_f32_cuda(q, k, v, g, b, w, state)
    B, Hk, T, K = q.shape
    HV, V = v.shape[1], v.shape[3]
    if T != 1:
        raise ValueError("fused_step takes one token")
    q, k, v, g, b, w = _operands(q, k, v, g, b, w)
    state = state.contiguous()
    new_state = torch.empty_like(state) if out_state is None else out_state
    out = torch.empty((B, HV, 1, V), device=q.device, dtype=torch.float32)
    sq, sv = _strides3(q), _strides3(v)
    for t in (k, g, b):
        if _strides3(t) != sq:
            raise ValueError("q, k, g, b must share one layout")
    if _strides3(w) != sv:
        raise ValueError("v and w must share one layout")
    a = C.StepArgs(_p(q), _p(k), _p(g), _p(b), _p(v), _p(w), _p(state), _p(new_state), _p(out),
                   B, Hk, HV, K, V, sq[0], sq[1], sv[0], sv[1], out.stride(0), out.stride(1), float(scale))
    if not C.check(C.lib().gdn2_recurrent_step_f32(ctypes.byref(a), _stream()), allow_not_applicable=True):
        return None
    return out, new_state


def fused_recurrent_forward(q, k, v, g, b, w, state, scale: float, out=None, in_place=False):
    """Per-token scan over T tokens in one launch.  Returns (out, new_state).
    g and b may have a last dim of 1 (one value per head and token)."""
    _check_f32_cuda(q, k, v, g, b, w, state)
    q, k, v, g, b, w = _operands(q, k, v, g, b, w)
    B, Hk, T, K = q.shape
    HV, V = v.shape[1], v.shape[3]
    state = state.contiguous()
    if out is None:
        out = torch.empty((B, HV, T, V), device=q.device, dtype=torch.float32)
    if T == 0:
        return out, (state if in_place else state.clone())
    new_state = state if in_place else torch.empty_like(state)
    sq, sv, so = _strides3(q), _strides3(v), _strides3(out)
    for t in (k, g, b):
        if _strides3(t) != sq:
            raise ValueError("q, k, g, b must share one layout")
    if _strides3(w) != sv:
        raise ValueError("v and w must share one layout")
    a = C.RecurrentArgs(_p(q), _p(k), _p(g), _p(b), _p(v), _p(w), _p(state), _p(new_state), _p(out),
                        B, Hk, HV, T, K, V, *sq, *sv, *so, float(scale))
    C.check(C.lib().gdn2_recurrent_fwd_f32(ctypes.byref(a), _stream()))
    return out, new_state


def fused_recurrent_gdn2(q, k, v, g, b, w, state=None, scale: float = 1.0, update_state: bool = True):
    """The reference's recurrent dispatch (src/kernel/fused_recurrent.rs:65-108):
    state None means zeros; with update_state a single token runs the fused
    step and longer inputs the scan, returning (out [B, HV, T, V], new state).
    With update_state False the state is only read: out = scale * q S, laid
    out [B, T, HV, V] as the reference's read-only branch permutes it, and the
    state comes back unchanged.  That branch runs the scan with k = 0 and
    g = 0, which leaves S exactly as it is (decay e^0 = 1, update 0 * v_new)
    while every token reads it."""
    _check_f32_cuda(q, k, v, g, b, w, state)
    B, Hk, T, K = q.shape
    HV, V = v.shape[1], v.shape[3]
    if state is None:
        state = torch.zeros((B, HV, K, V), device=q.device, dtype=torch.float32)
    if update_state:
        if T == 1:
            res = fused_step(q, k, v, g, b, w, state, scale)
            if res is not None:
                return res
        return fused_recurrent_forward(q, k, v, g, b, w, state, scale)
    zk = torch.zeros_like(q)
    out, _ = fused_recurrent_forward(q, zk, v, zk, zk, w, state, scale)
    return out.permute(0, 2, 1, 3), state


def chunk_args(q, k, v, g, b, w, state, out, scale, chunk_size, workspace=None):
    B, Hk, T, K = q.shape
    HV, V = v.shape[1], v.shape[3]
    sq, sv, so = _strides3(q), _strides3(v), _strides3(out)
    for t in (k, g, b):
        if _strides3(t) != sq:
            raise ValueError("q, k, g, b must share one layout")
    if _strides3(w) != sv:
        raise ValueError("v and w must share one layout")
    ws_ptr = None if workspace is None else _p(workspace)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    return C.ChunkArgs(_p(q), _p(k), _p(g), _p(b), _p(v), _p(w), _p(state), _p(out), B, Hk, HV, T, K, V,
                       *sq, *sv, *so, float(scale), int(chunk_size), ws_ptr, ws_bytes)


def chunk_workspace_bytes(q, k, v, g, b, w, state, out, scale, chunk_size) -> int:
    a = chunk_args(q, k, v, g, b, w, state, out, scale, chunk_size)
    return int(C.lib().gdn2_chunk_workspace_bytes(ctypes.byref(a)))


def chunk_wy_forward(q, k, v, g, b, w, state, scale: float, chunk_size: int = 64, out=None, workspace=None,
                     in_place=False, return_states=False):
    """Chunked forward over the whole sequence.  Returns (out, new_state),
    or None when the chunk kernels do not apply (K, V or chunk size outside
    their limits).  g and b may have a last dim of 1 (one value per head and
    token), as in the reference.

    return_states=True returns fused_chunk_forward's whole tuple
    (src/kernel/chunk_cube.rs:781-952): (out, new_state, v_new, states) with
    v_new [B*HV*NC, C, V] (the delta-rule values of each chunk of C =
    chunk_size tokens) and states [B*HV*NC, K, V] (the state entering each
    chunk).  chunk_size 64: NC = ceil(T/64) (rows past T are zero); a smaller
    chunk_size must divide T (the reference's C <= 64 and T % C == 0), NC =
    T/C; other chunk sizes return None."""
    _check_f32_cuda(q, k, v, g, b, w, state)
    q, k, v, g, b, w = _operands(q, k, v, g, b, w)
    B, Hk, T, K = q.shape
    HV, V = v.shape[1], v.shape[3]
    st = state.contiguous()
    if not in_place:
        st = st.clone()
    if out is None:
        out = torch.empty((B, HV, T, V), device=q.device, dtype=torch.float32)
    Cs = 64 if (not return_states or chunk_size == 64) else int(chunk_size)
    nblk = B * HV * ((T + 63) // 64 if Cs == 64 else (T // Cs if Cs > 0 else 0))
    if return_states:
        if Cs <= 0 or Cs > 64 or (Cs < 64 and T % Cs):
            return None  # the per-chunk tensors exist for chunk sizes up to 64 that divide T
        v_new = torch.empty((nblk, Cs, V), device=q.device, dtype=torch.float32)
        states = torch.empty((nblk, K, V), device=q.device, dtype=torch.float32)
    if T == 0:
        return (out, st, v_new, states) if return_states else (out, st)
    need = chunk_workspace_bytes(q, k, v, g, b, w, st, out, scale, chunk_size)
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    a = chunk_args(q, k, v, g, b, w, st, out, scale, chunk_size, workspace)
    if return_states:
        status = C.lib().gdn2_chunk_fwd_states_f32(ctypes.byref(a), v_new.data_ptr(), states.data_ptr(), _stream())
    else:
        status = C.lib().gdn2_chunk_fwd_f32(ctypes.byref(a), _stream())
    if not C.check(status, allow_not_applicable=True):
        return None
    return (out, st, v_new, states) if return_states else (out, st)


def chunk_wy_forward_train(q, k, v, g, b, w, state, scale: float, chunk_size: int = 64, out=None, workspace=None):
    """The training forward: (out, new_state, saved), the output and final
    state of chunk_wy_forward plus `saved`, a device buffer holding the
    quantities the backward takes (the reference's FusedBackwardInputs,
    src/kernel/chunk_adjoint_cube.rs:426-447), for chunk_wy_backward(...,
    saved=saved) on the same operands.  None when the chunked backward does
    not take these heads."""
    _check_f32_cuda(q, k, v, g, b, w, state)
    q, k, v, g, b, w = _operands(q, k, v, g, b, w)
    B, Hk, T, K = q.shape
    HV, V = v.shape[1], v.shape[3]
    st = state.contiguous().clone()
    if out is None:
        out = torch.empty((B, HV, T, V), device=q.device, dtype=torch.float32)
    fwd = chunk_args(q, k, v, g, b, w, st, out, scale, chunk_size)
    a = C.ChunkBwdArgs(fwd, None, None, None, None, None, None, None, None, None, None, 0)
    need = int(C.lib().gdn2_chunk_bwd_workspace_bytes(ctypes.byref(a)))
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    a.workspace, a.workspace_bytes = _p(workspace), workspace.numel() * workspace.element_size()
    if not C.check(C.lib().gdn2_chunk_fwd_train_f32(ctypes.byref(a), _stream()), allow_not_applicable=True):
        return None
    return out, st, workspace


def chunk_wy_backward(q, k, v, g, b, w, state0, d_out, scale: float, chunk_size: int = 64, d_state=None,
                      workspace=None, saved=None):
    """Gradients of the chunked forward (fused_chunk_backward,
    src/kernel/chunk_adjoint_cube.rs:464-707): for
    L = <d_out, out> + <d_state, S_T> returns dict dq, dk, dg, db (shapes of
    q, k, g, b), dv, dw (shapes of v, w) and dS0, or None when the chunk
    kernels do not apply.  dq, dk, dg, db take q's layout and dv, dw v's; dg
    and db of a g or b with a last dim of 1 are summed over the channels.
    With `saved` (from chunk_wy_forward_train on the same operands) the
    forward's per-chunk quantities are taken from it instead of recomputed
    (state0 is then not read)."""
    _check_f32_cuda(q, k, v, g, b, w, state0, d_out)
    g_in, b_in = g, b
    q, k, v, g, b, w = _operands(q, k, v, g, b, w)
    d_out = _channels_contiguous(d_out)
    B, Hk, T, K = q.shape
    HV, V = v.shape[1], v.shape[3]
    st = state0.contiguous()
    grads = {n: torch.empty_strided(t.shape, t.stride(), device=t.device, dtype=torch.float32)
             for n, t in (("dq", q), ("dk", q), ("dg", q), ("db", q), ("dv", v), ("dw", v))}
    grads["dS0"] = torch.empty((B, HV, K, V), device=q.device, dtype=torch.float32)
    ds = None if d_state is None else d_state.contiguous()
    if T == 0:  # no tokens: only the state gradient passes through
        grads["dS0"] = ds.clone() if ds is not None else torch.zeros_like(grads["dS0"])
        grads["dg"], grads["db"] = _reduce_like(grads["dg"], g_in), _reduce_like(grads["db"], b_in)
        return grads
    fwd = chunk_args(q, k, v, g, b, w, st, d_out, scale, chunk_size)
    a = C.ChunkBwdArgs(fwd, _p(d_out), _p(ds), *(_p(grads[n]) for n in ("dq", "dk", "dg", "db", "dv", "dw", "dS0")),
                       None, 0)
    if saved is not None:
        workspace = saved
    need = int(C.lib().gdn2_chunk_bwd_workspace_bytes(ctypes.byref(a)))
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        if saved is not None:
            raise ValueError("saved holds fewer bytes than this backward's workspace: not from these operands")
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    a.workspace, a.workspace_bytes = _p(workspace), workspace.numel() * workspace.element_size()
    fn = C.lib().gdn2_chunk_bwd_saved_f32 if saved is not None else C.lib().gdn2_chunk_bwd_f32
    if not C.check(fn(ctypes.byref(a), _stream()), allow_not_applicable=True):
        return None
    grads["dg"], grads["db"] = _reduce_like(grads["dg"], g_in), _reduce_like(grads["db"], b_in)
    return grads


def fused_recurrent_backward(q, k, v, g, b, w, state0, d_out, scale: float, d_state=None, workspace=None):
    """Gradients of the per-token scan (fused_recurrent_forward) for any (K, V)
    the scan backward kernel takes: for L = <d_out, out> + <d_state, S_T>
    returns dict dq, dk, dg, db, dv, dw, dS0 (layouts as chunk_wy_backward),
    or None outside its limits.  state0 None means zeros."""
    _check_f32_cuda(q, k, v, g, b, w, state0, d_out)
    g_in, b_in = g, b
    q, k, v, g, b, w = _operands(q, k, v, g, b, w)
    d_out = _channels_contiguous(d_out)
    B, Hk, T, K = q.shape
    HV, V = v.shape[1], v.shape[3]
    st = None if state0 is None else state0.contiguous()
    grads = {n: torch.empty_strided(t.shape, t.stride(), device=t.device, dtype=torch.float32)
             for n, t in (("dq", q), ("dk", q), ("dg", q), ("db", q), ("dv", v), ("dw", v))}
    grads["dS0"] = torch.empty((B, HV, K, V), device=q.device, dtype=torch.float32)
    ds = None if d_state is None else d_state.contiguous()
    if T == 0:  # no tokens: only the state gradient passes through
        grads["dS0"] = ds.clone() if ds is not None else torch.zeros_like(grads["dS0"])
        grads["dg"], grads["db"] = _reduce_like(grads["dg"], g_in), _reduce_like(grads["db"], b_in)
        return grads
    sq, sv, so = _strides3(q), _strides3(v), _strides3(d_out)
    fwd = C.RecurrentArgs(_p(q), _p(k), _p(g), _p(b), _p(v), _p(w), _p(st), None, None, B, Hk, HV, T, K, V,
                          *sq, *sv, *so, float(scale))
    a = C.RecurrentBwdArgs(fwd, _p(d_out), _p(ds), *(_p(grads[n]) for n in ("dq", "dk", "dg", "db", "dv", "dw", "dS0")),
                           None, 0)
    need = int(C.lib().gdn2_recurrent_bwd_workspace_bytes(ctypes.byref(a)))
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    a.workspace, a.workspace_bytes = _p(workspace), workspace.numel() * workspace.element_size()
    if not C.check(C.lib().gdn2_recurrent_bwd_f32(ctypes.byref(a), _stream()), allow_not_applicable=True):
        return None
    grads["dg"], grads["db"] = _reduce_like(grads["dg"], g_in), _reduce_like(grads["db"], b_in)
    return grads


def decode_args(raw: dict, params: dict, state, conv_in, conv_out, out, *, num_heads, num_v_heads, head_dim,
                head_v_dim, scale, min_decay=None, norm_eps=1e-5, use_short_conv=True, allow_neg_eigval=False):
    """Build the gdn2_decode_args block (the LayerParams it points to is
    kept alive as an attribute of the returned struct)."""
    B = raw["q_raw"].shape[0]
    lp = C.LayerParams(_p(params.get("q_conv_w")), _p(params.get("k_conv_w")), _p(params.get("v_conv_w")),
                       _p(params["a_log"]), _p(params["dt_bias"]), _p(params.get("decay_factors")),
                       _p(params["o_norm_weight"]), float(min_decay or 0.0), float(norm_eps),
                       int(use_short_conv), int(allow_neg_eigval))
    ci = conv_in if conv_in is not None else (None, None, None)
    co = conv_out if conv_out is not None else (None, None, None)
    a = C.DecodeArgs(_p(raw["q_raw"]), _p(raw["k_raw"]), _p(raw["f_raw"]), _p(raw["b_raw"]), _p(raw["v_raw"]),
                     _p(raw["w_raw"]), _p(raw["gate"]), _p(ci[0]), _p(ci[1]), _p(ci[2]), _p(co[0]), _p(co[1]),
                     _p(co[2]), _p(state), _p(out), B, num_heads, num_v_heads, head_dim, head_v_dim, float(scale),
                     ctypes.pointer(lp))
    a._keep = lp
    return a


def decode_fused(raw: dict, params: dict, state, conv_in, conv_out, *, num_heads, num_v_heads, head_dim,
                 head_v_dim, scale, min_decay=None, norm_eps=1e-5, use_short_conv=True, allow_neg_eigval=False,
                 out=None):
    """Fused single-token decode.  raw: q_raw, k_raw, f_raw, b_raw [B, kd];
    v_raw, w_raw, gate [B, vd].  params: q/k/v_conv_w, a_log, dt_bias,
    decay_factors (optional), o_norm_weight.  conv_in: (q, k, v) caches
    [B, 3, kd|vd] or None (no prior state); conv_out: output caches.
    Updates state in place; returns out [B, vd] (input of o_proj)."""
    B = raw["q_raw"].shape[0]
    vd = num_v_heads * head_v_dim
    if out is None:
        out = torch.empty((B, vd), device=raw["q_raw"].device, dtype=torch.float32)
    a = decode_args(raw, params, state, conv_in, conv_out, out, num_heads=num_heads, num_v_heads=num_v_heads,
                    head_dim=head_dim, head_v_dim=head_v_dim, scale=scale, min_decay=min_decay, norm_eps=norm_eps,
                    use_short_conv=use_short_conv, allow_neg_eigval=allow_neg_eigval)
    C.check(C.lib().gdn2_decode_fused_f32(ctypes.byref(a), _stream()))
    return out


# -- the reference's standalone operators (src/lib.rs:58-62) -------------------

def short_conv_1d(x, weight, cache=None):
    """short_conv_1d (src/short_conv.rs:22-65): x [B, T, C], weight [C, 4],
    cache [B, 3, C] or None (the first token repeated as padding).  Returns
    (silu(causal conv of 4 taps) [B, T, C], new cache [B, 3, C])."""
    _check_f32_cuda(x, weight, cache)
    x, weight = x.contiguous(), weight.contiguous()
    cache = None if cache is None else cache.contiguous()
    B, T, Cn = x.shape
    if tuple(weight.shape) != (Cn, 4) or (cache is not None and tuple(cache.shape) != (B, 3, Cn)):
        raise ValueError("short_conv_1d: weight must be [C, 4] and cache [B, 3, C]")
    out = torch.empty_like(x)
    new_cache = torch.empty((B, 3, Cn), device=x.device, dtype=torch.float32)
    C.check(C.lib().gdn2_short_conv_f32(_p(x), _p(weight), _p(cache), _p(out), _p(new_cache), B, T, Cn, _stream()))
    return out, new_cache


def l2_normalize(x, eps: float = 1e-6):
    """l2_normalize / l2_normalize_4d (src/l2norm.rs:4-16): x / sqrt(sum x^2 +
    eps) along the last dimension, any leading shape."""
    _check_f32_cuda(x)
    x = x.contiguous()
    y = torch.empty_like(x)
    n = x.shape[-1] if x.dim() else 1
    C.check(C.lib().gdn2_l2_normalize_f32(_p(x), _p(y), x.numel() // max(n, 1), n, float(eps), _stream()))
    return y


l2_normalize_4d = l2_normalize


def rms_norm_gate_per_head(x, gate, weight, eps: float):
    """rms_norm_gate_per_head (src/module.rs:501-517): x, gate [B, T, HV, V],
    weight [V]: x / sqrt(mean_V x^2 + eps) * weight * silu(gate)."""
    _check_f32_cuda(x, gate, weight)
    x, gate, weight = x.contiguous(), gate.contiguous(), weight.contiguous()
    if gate.shape != x.shape or weight.numel() != x.shape[-1]:
        raise ValueError("rms_norm_gate_per_head: gate must match x and weight must have x's last dim")
    y = torch.empty_like(x)
    V = x.shape[-1]
    C.check(C.lib().gdn2_rms_norm_gate_f32(_p(x), _p(gate), _p(weight), _p(y), x.numel() // V, V, float(eps),
                                           _stream()))
    return y

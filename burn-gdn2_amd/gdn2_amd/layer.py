"""The GDN-2 layer: Python mirror of burn-gdn2's public surface over the C ABI
of include/gdn2_layer.h.

  Gdn2Config      src/config.rs:23-130 (fields, Default, validate)
  GatedDeltaNet2  src/module.rs:93-495 (new, forward, forward_train, project)
  Gdn2State       src/module.rs:30-63
  Gdn2Grads       the parameter gradients that burn's autodiff returns
                  (tests/autodiff.rs:153-205), from GatedDeltaNet2.backward

Parameters live in device memory owned by the library; x and the outputs
are float32 torch device tensors [B, T, hidden_size].  Every call runs the
library's HIP kernels and hipBLASLt GEMMs (rocBLAS for any shape hipBLASLt
has no algorithm for) on torch's current stream; there is no CPU path.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import numpy as np

from . import _capi as C

_MODES = {"fused_recurrent": C.MODE_FUSED_RECURRENT, "chunk": C.MODE_CHUNK}
_GVA_LAYOUTS = {"head_repeat": C.GVA_HEAD_REPEAT, "reference": C.GVA_REFERENCE}


def _stream():
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _msg() -> str:
    return C.lib().gdn2_last_error().decode(errors="replace")


@dataclass
class Gdn2Config:
    """Gdn2Config (src/config.rs:23-58); `mode` is "fused_recurrent" or "chunk".
    `gva_layout` (not a Gdn2Config field) is "head_repeat" (value head hv
    reads key head hv / rep at every time, so decode reproduces prefill) or
    "reference" (the reference tensor path's unsqueeze/repeat/reshape,
    src/module.rs:456-468: value head h rep + a at time t reads key head h at
    time (a T + t) / rep of the same call)."""
    hidden_size: int = 2048
    num_heads: int = 16
    head_dim: int = 128
    expand_v: float = 1.0
    num_v_heads: Optional[int] = None
    use_short_conv: bool = True
    allow_neg_eigval: bool = False
    norm_eps: float = 1e-5
    mode: str = "fused_recurrent"
    chunk_size: int = 64
    min_decay: Optional[float] = None
    gva_layout: str = "head_repeat"

    def to_c(self) -> C.Config:
        if self.mode not in _MODES:
            raise ValueError(f"mode must be one of {sorted(_MODES)}, got {self.mode!r}")
        if self.gva_layout not in _GVA_LAYOUTS:
            raise ValueError(f"gva_layout must be one of {sorted(_GVA_LAYOUTS)}, got {self.gva_layout!r}")
        return C.Config(int(self.hidden_size), int(self.num_heads), int(self.head_dim), float(self.expand_v),
                        0 if self.num_v_heads is None else int(self.num_v_heads), int(bool(self.use_short_conv)),
                        int(bool(self.allow_neg_eigval)), float(self.norm_eps), _MODES[self.mode],
                        int(self.chunk_size), int(self.min_decay is not None), float(self.min_decay or 0.0),
                        _GVA_LAYOUTS[self.gva_layout])

    def validate(self) -> None:
        """Gdn2Config::validate (src/config.rs:71-111): raises ValueError with
        the reference's panic message."""
        c = self.to_c()
        st = C.lib().gdn2_config_validate(ctypes.byref(c))
        if st != C.GDN2_OK:
            raise ValueError(_msg())

    @property
    def hv(self) -> int:
        return self.num_v_heads or self.num_heads

    @property
    def v_head(self) -> int:
        return int(np.float32(self.head_dim) * np.float32(self.expand_v))

    @property
    def kd(self) -> int:
        return self.num_heads * self.head_dim

    @property
    def hq(self) -> int:
        """Key-side heads of the recurrence's q, k, g, b: num_heads, or the
        value heads in the reference's GVA layout."""
        return self.hv if self.gva_layout == "reference" else self.num_heads

    @property
    def vd(self) -> int:
        return self.hv * self.v_head


def param_names() -> Tuple[str, ...]:
    L = C.lib()
    return tuple(L.gdn2_param_name(i).decode() for i in range(L.gdn2_param_count()))


def param_shape(cfg: Gdn2Config, name: str) -> Tuple[int, ...]:
    """Shape of parameter `name` ((), when absent in this config)."""
    rows, cols = C._i64(), C._i64()
    n = C.lib().gdn2_param_shape(ctypes.byref(cfg.to_c()), name.encode(), ctypes.byref(rows), ctypes.byref(cols))
    if n < 0:
        raise KeyError(name)
    if n == 0:
        return ()
    return (rows.value,) if cols.value == 1 and name in _VECTORS else (rows.value, cols.value)


_VECTORS = {"g_proj_1_bias", "a_log", "dt_bias", "o_norm_weight"}


def init_param(cfg: Gdn2Config, name: str, seed: int = 1337) -> Optional[np.ndarray]:
    """Host-side initial value of one parameter (GatedDeltaNet2::new's
    initialisers, src/module.rs:121-187); None when absent.  CPU only."""
    shape = param_shape(cfg, name)
    if not shape:
        return None
    out = np.empty(shape, np.float32)
    st = C.lib().gdn2_param_init(ctypes.byref(cfg.to_c()), ctypes.c_uint64(seed), name.encode(),
                                 out.ctypes.data_as(ctypes.c_void_p), out.size)
    C.check(st)
    return out


def init_params(cfg: Gdn2Config, seed: int = 1337) -> Dict[str, Optional[np.ndarray]]:
    return {n: init_param(cfg, n, seed) for n in param_names()}


class Gdn2State:
    """Option<Gdn2State> for one layer and batch (src/module.rs:30-63).
    A fresh object is empty (None); `zeros` gives Gdn2State::zeros."""
    RECURRENT, CONV_Q, CONV_K, CONV_V = C.STATE_RECURRENT, C.STATE_CONV_Q, C.STATE_CONV_K, C.STATE_CONV_V

    def __init__(self, layer: "GatedDeltaNet2", batch: int):
        self._layer = layer  # keeps the layer alive while the state exists
        h = ctypes.c_void_p()
        C.check(C.lib().gdn2_state_create(layer._h, int(batch), ctypes.byref(h)))
        self._h = h

    @classmethod
    def zeros(cls, layer: "GatedDeltaNet2", batch: int) -> "Gdn2State":
        s = cls(layer, batch)
        C.check(C.lib().gdn2_state_set_zeros(s._h))
        return s

    def close(self):
        if getattr(self, "_h", None):
            C.lib().gdn2_state_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def is_some(self) -> bool:
        return bool(C.lib().gdn2_state_is_some(self._h))

    @property
    def batch(self) -> int:
        return int(C.lib().gdn2_state_batch(self._h))

    def _shape(self, which):
        cfg, B = self._layer.config, self.batch
        if which == self.RECURRENT:
            return (B, cfg.hv, cfg.head_dim, cfg.v_head)
        return (B, 3, cfg.vd if which == self.CONV_V else cfg.kd)

    def read(self, which: int) -> np.ndarray:
        out = np.empty(self._shape(which), np.float32)
        C.check(C.lib().gdn2_state_read(self._h, which, out.ctypes.data_as(ctypes.c_void_p), out.size))
        return out

    def write(self, which: int, value) -> None:
        a = np.ascontiguousarray(value, np.float32)
        if a.shape != self._shape(which):
            raise ValueError(f"expected shape {self._shape(which)}, got {a.shape}")
        C.check(C.lib().gdn2_state_write(self._h, which, a.ctypes.data_as(ctypes.c_void_p), a.size))

    # -- interchange (safetensors; tensor names are the reference's fields) --
    def to_bytes(self) -> bytes:
        """The state as safetensors bytes: "recurrent", "conv_q", "conv_k",
        "conv_v" (src/module.rs:30-40) plus a __metadata__ block."""
        n = ctypes.c_size_t()
        C.check(C.lib().gdn2_state_serialize(self._h, None, 0, ctypes.byref(n)))
        buf = ctypes.create_string_buffer(n.value)
        C.check(C.lib().gdn2_state_serialize(self._h, buf, n.value, ctypes.byref(n)))
        return buf.raw[:n.value]

    def load_bytes(self, data: bytes) -> None:
        """Fill this state from safetensors bytes (shapes must match)."""
        buf = ctypes.create_string_buffer(bytes(data), len(data))
        C.check(C.lib().gdn2_state_deserialize(self._h, buf, len(data)))

    @classmethod
    def from_bytes(cls, layer: "GatedDeltaNet2", data: bytes) -> "Gdn2State":
        """A new state of `layer` from safetensors bytes; the batch comes from
        the "recurrent" tensor's shape."""
        import json

        hn = int.from_bytes(data[:8], "little")
        batch = json.loads(data[8:8 + hn])["recurrent"]["shape"][0]
        s = cls(layer, batch)
        s.load_bytes(data)
        return s

    def save(self, path: str) -> None:
        with open(path, "wb") as fh:
            fh.write(self.to_bytes())

    @classmethod
    def load(cls, layer: "GatedDeltaNet2", path: str) -> "Gdn2State":
        with open(path, "rb") as fh:
            return cls.from_bytes(layer, fh.read())

    @property
    def recurrent(self) -> np.ndarray:
        return self.read(self.RECURRENT)

    @property
    def conv_q(self) -> np.ndarray:
        return self.read(self.CONV_Q)

    @property
    def conv_k(self) -> np.ndarray:
        return self.read(self.CONV_K)

    @property
    def conv_v(self) -> np.ndarray:
        return self.read(self.CONV_V)


class Gdn2Grads:
    """Gradients of every parameter of one layer, in device buffers owned by
    the library (zero on creation).  `get(name)` returns a host copy in the
    parameter's shape."""

    def __init__(self, layer: "GatedDeltaNet2"):
        self._layer = layer
        h = ctypes.c_void_p()
        C.check(C.lib().gdn2_layer_grads_create(layer._h, ctypes.byref(h)))
        self._h = h

    def close(self):
        if getattr(self, "_h", None):
            C.lib().gdn2_layer_grads_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def zero(self) -> None:
        C.check(C.lib().gdn2_layer_grads_zero(self._h, _stream()))

    def get(self, name: str) -> Optional[np.ndarray]:
        shape = param_shape(self._layer.config, name)
        if not shape:
            return None
        out = np.empty(shape, np.float32)
        C.check(C.lib().gdn2_layer_grads_get(self._h, name.encode(), out.ctypes.data_as(ctypes.c_void_p), out.size))
        return out

    def as_dict(self) -> Dict[str, Optional[np.ndarray]]:
        return {n: self.get(n) for n in param_names()}


class Gdn2Saved:
    """Activations kept by forward_train for the backward (one object per
    batch and sequence length; see GatedDeltaNet2.forward_train)."""

    def __init__(self, layer: "GatedDeltaNet2", batch: int, seq_len: int):
        self._layer = layer
        h = ctypes.c_void_p()
        C.check(C.lib().gdn2_layer_saved_create(layer._h, int(batch), int(seq_len), ctypes.byref(h)))
        self._h = h
        self.shape = (int(batch), int(seq_len))

    def close(self):
        if getattr(self, "_h", None):
            C.lib().gdn2_layer_saved_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _forward_train_fn():
    import torch

    class _ForwardTrain(torch.autograd.Function):
        @staticmethod
        def forward(ctx, x, layer):
            ctx.layer = layer
            ctx.save_for_backward(x)
            ctx.acts = Gdn2Saved(layer, x.shape[0], x.shape[1])
            return layer.forward_train(x, saved=ctx.acts)

        @staticmethod
        def backward(ctx, d_out):
            (x,) = ctx.saved_tensors
            layer = ctx.layer
            if layer.grads is None:
                layer.grads = Gdn2Grads(layer)
            dx, _, _ = layer.backward(x, d_out, saved=ctx.acts, grads=layer.grads, accumulate=True)
            ctx.acts.close()
            return dx, None

    return _ForwardTrain


class GatedDeltaNet2:
    """GatedDeltaNet2 (src/module.rs:93-495) on the current HIP device."""

    def __init__(self, cfg: Gdn2Config, seed: int = 1337):
        cfg.validate()
        self.config = cfg
        h = ctypes.c_void_p()
        C.check(C.lib().gdn2_layer_create(ctypes.byref(cfg.to_c()), ctypes.c_uint64(seed), ctypes.byref(h)))
        self._h = h
        self.grads: Optional[Gdn2Grads] = None  # filled by forward_train_autograd's backward

    def close(self):
        if getattr(self, "grads", None) is not None:
            self.grads.close()
            self.grads = None
        if getattr(self, "_h", None):
            C.lib().gdn2_layer_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- parameters ---------------------------------------------------------
    def param(self, name: str) -> Optional[np.ndarray]:
        shape = param_shape(self.config, name)
        if not shape:
            return None
        out = np.empty(shape, np.float32)
        C.check(C.lib().gdn2_layer_get_param(self._h, name.encode(), out.ctypes.data_as(ctypes.c_void_p), out.size))
        return out

    def set_param(self, name: str, value) -> None:
        a = np.ascontiguousarray(value, np.float32)
        shape = param_shape(self.config, name)
        if a.shape != shape and a.size != int(np.prod(shape or (0,))):
            raise ValueError(f"{name}: expected shape {shape}, got {a.shape}")
        C.check(C.lib().gdn2_layer_set_param(self._h, name.encode(), a.ctypes.data_as(ctypes.c_void_p), a.size))

    def params(self) -> Dict[str, Optional[np.ndarray]]:
        return {n: self.param(n) for n in param_names()}

    def load_params(self, params: Dict[str, Optional[np.ndarray]]) -> None:
        for n, a in params.items():
            if a is not None:
                self.set_param(n, a)

    # -- forward ------------------------------------------------------------
    def _check_x(self, x):
        import torch

        if x.dtype != torch.float32 or not x.is_cuda or x.dim() != 3:
            raise TypeError("x must be a float32 device tensor [B, T, hidden_size]")
        if x.shape[2] != self.config.hidden_size:
            # GatedDeltaNet2::validate (src/module.rs:198-206)
            raise ValueError(f"GatedDeltaNet2: expected hidden_states with last dim {self.config.hidden_size} "
                             f"but got {x.shape[2]}. Check that the model hidden_size matches your input.")
        return x.contiguous()

    def forward_train(self, x, saved: Optional["Gdn2Saved"] = None):
        """forward_train (src/module.rs:326-375): [B, T, D] -> [B, T, D].
        With `saved` (a Gdn2Saved of x's batch and length) the activations
        the backward needs are kept in it."""
        import torch

        x = self._check_x(x)
        out = torch.empty_like(x)
        if saved is None:
            C.check(C.lib().gdn2_layer_forward_train_f32(self._h, x.data_ptr(), x.shape[0], x.shape[1],
                                                         out.data_ptr(), _stream()))
        else:
            C.check(C.lib().gdn2_layer_forward_train_saved_f32(self._h, x.data_ptr(), x.shape[0], x.shape[1],
                                                               out.data_ptr(), saved._h, _stream()))
        return out

    def forward(self, x, state: Optional[Gdn2State] = None):
        """forward(x, &mut state, update_state = true) (src/module.rs:224-316).
        Returns (out [B, T, D], state); a None state is created empty and
        filled, as the reference's `get_or_insert_with`."""
        import torch

        x = self._check_x(x)
        if state is None:
            state = Gdn2State(self, x.shape[0])
        out = torch.empty_like(x)
        C.check(C.lib().gdn2_layer_forward_f32(self._h, x.data_ptr(), x.shape[0], x.shape[1], state._h,
                                               out.data_ptr(), _stream()))
        return out, state

    def project(self, x, state: Optional[Gdn2State] = None) -> Dict[str, "torch.Tensor"]:
        """project (src/module.rs:381-495): q, k, g, b as the recurrence takes
        them, [B, H, T, K] under head repeat (the key heads, not repeated) or
        [B, HV, T, K] in the reference's GVA layout (what its project
        returns); v, w [B, HV, T, V] and gate [B, T, HV, V]."""
        import torch

        x = self._check_x(x)
        cfg = self.config
        B, T = x.shape[:2]
        o = {n: torch.empty((B, cfg.hq, T, cfg.head_dim), device=x.device) for n in ("q", "k", "g", "b")}
        o.update({n: torch.empty((B, cfg.hv, T, cfg.v_head), device=x.device) for n in ("v", "w")})
        o["gate"] = torch.empty((B, T, cfg.hv, cfg.v_head), device=x.device)
        C.check(C.lib().gdn2_layer_project_f32(self._h, x.data_ptr(), B, T, state._h if state is not None else None,
                                               *(o[n].data_ptr() for n in ("q", "k", "g", "b", "v", "w", "gate")),
                                               _stream()))
        return o

    # -- backward -----------------------------------------------------------
    def backward(self, x, d_out, state: Optional[Gdn2State] = None, d_state: Optional[Gdn2State] = None,
                 grads: Optional[Gdn2Grads] = None, accumulate: bool = False, want_dx: bool = True,
                 want_d_state: bool = False, saved: Optional[Gdn2Saved] = None):
        """Gradients of <d_out, out> + <d_state, state after the call> for
        forward(x, state) (state None or empty: forward_train).  `state` is
        the state BEFORE that call and is not modified; `saved`, filled by
        forward_train(x, saved=...), replaces the recomputation.  Returns
        (dx or None, grads, d_state_in or None); parameter gradients go into
        `grads` (a new Gdn2Grads when None), added to it with accumulate."""
        import torch

        x = self._check_x(x)
        if d_out.shape != x.shape or d_out.dtype != torch.float32 or not d_out.is_cuda:
            raise TypeError("d_out must be a float32 device tensor shaped like x")
        d_out = d_out.contiguous()
        B, T = x.shape[:2]
        if grads is None:
            grads = Gdn2Grads(self)
        dx = torch.empty_like(x) if want_dx else None
        d_state_in = Gdn2State(self, B) if want_d_state else None
        C.check(C.lib().gdn2_layer_backward_f32(
            self._h, x.data_ptr(), B, T, state._h if state is not None else None,
            saved._h if saved is not None else None, d_out.data_ptr(),
            d_state._h if d_state is not None else None, dx.data_ptr() if dx is not None else None,
            d_state_in._h if d_state_in is not None else None, grads._h, int(bool(accumulate)), _stream()))
        return dx, grads, d_state_in

    def forward_train_autograd(self, x):
        """forward_train as a torch autograd node: `loss.backward()` adds the
        parameter gradients to `self.grads` (created on first use, as burn's
        Gradients) and propagates dx to x."""
        return _forward_train_fn().apply(x, self)

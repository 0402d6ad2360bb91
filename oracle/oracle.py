"""ctypes front end of the CPU oracle (oracle/gdn2_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.  Each function
names the reference code it restates; the C file documents how each one is
pinned.

Array conventions (numpy, C-contiguous):
  q, k, g, b  [B, Hk, T, K]   (g, b may have last dim 1)
  v, w        [B, HV, T, V]
  S           [B, HV, K, V]
  out         [B, HV, T, V]
Value head hv reads key head hv // (HV // Hk).

layer_backward_f64 (the layer's adjoint, in numpy on double values with the
scan parts in C) is pinned by central finite differences of the C layer
forward in tests/test_oracle_layer_bwd.py.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libgdn2_oracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_vp = ctypes.c_void_p


def build() -> str:
    """Compile the oracle with its Makefile (gcc, OpenMP)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        i, d = ctypes.c_int, ctypes.c_double
        L.gdn2o_recurrent_f64.argtypes = [_vp] * 7 + [i] * 8 + [d, _vp, _vp]
        L.gdn2o_recurrent_f32.argtypes = [_vp] * 7 + [i] * 8 + [d, _vp, _vp]
        L.gdn2o_recurrent_bwd_f64.argtypes = [_vp] * 9 + [i] * 8 + [d] + [_vp] * 7
        L.gdn2o_recurrent_bwd_d.argtypes = [_vp] * 9 + [i] * 8 + [d] + [_vp] * 7
        L.gdn2o_scan_d.argtypes = [_vp] * 7 + [i] * 6 + [d, _vp]
        L.gdn2o_chunk_wy_f32.argtypes = [_vp] * 7 + [i] * 8 + [d, i, _vp, _vp]
        L.gdn2o_short_conv.argtypes = [_vp, _vp, _vp, i, i, i, _vp, _vp]
        L.gdn2o_l2norm_rows.argtypes = [_vp, ctypes.c_long, i, d]
        L.gdn2o_rmsnorm_gate.argtypes = [_vp, _vp, _vp, ctypes.c_long, i, d, _vp]
        L.gdn2o_layer_forward.argtypes = [_vp, _vp, _vp, i, i, i] + [_vp] * 13
        L.gdn2o_layer_from_raw.argtypes = [_vp, _vp] + [_vp] * 7 + [i, i, i] + [_vp] * 12
        L.gdn2o_num_threads.restype = i
        L.gdn2o_set_num_threads.argtypes = [i]
        _lib = L
    return _lib


def num_threads() -> int:
    return lib().gdn2o_num_threads()


def set_num_threads(n: int) -> None:
    lib().gdn2o_set_num_threads(int(n))


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _scan_shapes(q, k, v, g, b, w):
    B, Hk, T, K = q.shape
    HV, V = v.shape[1], v.shape[3]
    assert k.shape == q.shape and w.shape == v.shape
    assert v.shape[0] == B and v.shape[2] == T
    assert HV % Hk == 0
    gdim, bdim = g.shape[3], b.shape[3]
    assert g.shape[:3] == (B, Hk, T) and b.shape[:3] == (B, Hk, T)
    assert gdim in (1, K) and bdim in (1, K)
    return B, HV, Hk, T, K, V, gdim, bdim


def recurrent_f64(q, k, v, g, b, w, S0=None, scale=1.0):
    """Per-token scan in double (src/kernel/fused_recurrent.rs:27-52)."""
    q, k, v, g, b, w = (_c(a, np.float32) for a in (q, k, v, g, b, w))
    B, HV, Hk, T, K, V, gdim, bdim = _scan_shapes(q, k, v, g, b, w)
    S0 = None if S0 is None else _c(S0, np.float64)
    out = np.empty((B, HV, T, V), np.float64)
    S = np.empty((B, HV, K, V), np.float64)
    lib().gdn2o_recurrent_f64(*(_ptr(a) for a in (q, k, v, g, b, w, S0)), B, HV, Hk, T, K, V, gdim, bdim,
                              float(scale), _ptr(out), _ptr(S))
    return out, S


def recurrent_bwd_f64(q, k, v, g, b, w, d_out, S0=None, d_ST=None, scale=1.0):
    """Adjoint of the per-token scan in double: gradients of
    L = sum(d_out * out) + sum(d_ST * S_T) (the gradients the reference's
    training path takes through autodiff of the same scan, tests/autodiff.rs:153-206;
    the seven outputs of src/kernel/chunk_adjoint_cube.rs:464-707).
    Returns dict dq, dk, dg, db (key-head shapes of q, k, g, b), dv, dw, dS0."""
    q, k, v, g, b, w = (_c(a, np.float32) for a in (q, k, v, g, b, w))
    B, HV, Hk, T, K, V, gdim, bdim = _scan_shapes(q, k, v, g, b, w)
    S0 = None if S0 is None else _c(S0, np.float64)
    d_out = _c(d_out, np.float64)
    assert d_out.shape == (B, HV, T, V)
    d_ST = None if d_ST is None else _c(d_ST, np.float64)
    r = {"dq": np.empty(q.shape), "dk": np.empty(k.shape), "dg": np.empty(g.shape), "db": np.empty(b.shape),
         "dv": np.empty(v.shape), "dw": np.empty(w.shape), "dS0": np.empty((B, HV, K, V))}
    lib().gdn2o_recurrent_bwd_f64(*(_ptr(a) for a in (q, k, v, g, b, w, S0, d_out, d_ST)), B, HV, Hk, T, K, V,
                                  gdim, bdim, float(scale), *(_ptr(r[n]) for n in ("dq", "dk", "dg", "db", "dv",
                                                                                   "dw", "dS0")))
    return r


def recurrent_f32(q, k, v, g, b, w, S0=None, scale=1.0):
    """Per-token scan with the reference's f32 op order (src/kernel/fused_recurrent.rs:25-52)."""
    q, k, v, g, b, w = (_c(a, np.float32) for a in (q, k, v, g, b, w))
    B, HV, Hk, T, K, V, gdim, bdim = _scan_shapes(q, k, v, g, b, w)
    S0 = None if S0 is None else _c(S0, np.float32)
    out = np.empty((B, HV, T, V), np.float32)
    S = np.empty((B, HV, K, V), np.float32)
    lib().gdn2o_recurrent_f32(*(_ptr(a) for a in (q, k, v, g, b, w, S0)), B, HV, Hk, T, K, V, gdim, bdim,
                              float(scale), _ptr(out), _ptr(S))
    return out, S


def chunk_wy_f32(q, k, v, g, b, w, S0=None, scale=1.0, chunk_size=64):
    """Chunked WY forward, 16-tile log-space decay, f32 (src/forward.rs:44-278)."""
    q, k, v, g, b, w = (_c(a, np.float32) for a in (q, k, v, g, b, w))
    B, HV, Hk, T, K, V, gdim, bdim = _scan_shapes(q, k, v, g, b, w)
    S0 = None if S0 is None else _c(S0, np.float32)
    out = np.empty((B, HV, T, V), np.float32)
    S = np.empty((B, HV, K, V), np.float32)
    lib().gdn2o_chunk_wy_f32(*(_ptr(a) for a in (q, k, v, g, b, w, S0)), B, HV, Hk, T, K, V, gdim, bdim,
                             float(scale), int(chunk_size), _ptr(out), _ptr(S))
    return out, S


def short_conv(x, wconv, cache=None):
    """Causal depthwise conv k=4 + SiLU (src/short_conv.rs:22-65). x [B,T,C]."""
    x = _c(x, np.float64)
    wconv = _c(wconv, np.float32)
    B, T, C = x.shape
    assert wconv.shape == (C, 4)
    cache = None if cache is None else _c(cache, np.float64)
    y = np.empty((B, T, C), np.float64)
    nc = np.empty((B, 3, C), np.float64)
    lib().gdn2o_short_conv(_ptr(x), _ptr(wconv), _ptr(cache), B, T, C, _ptr(y), _ptr(nc))
    return y, nc


def l2norm(x, eps=1e-6):
    """x / sqrt(sum x^2 + eps) over the last dim (src/l2norm.rs:13-16)."""
    y = np.array(x, dtype=np.float64, order="C", copy=True)
    n = y.shape[-1]
    lib().gdn2o_l2norm_rows(_ptr(y), y.size // n, n, float(eps))
    return y


def rmsnorm_gate(x, gate, weight, eps):
    """x / sqrt(mean x^2 + eps) * weight * silu(gate) (src/module.rs:501-517)."""
    x = _c(x, np.float64)
    gate = _c(gate, np.float64)
    weight = _c(weight, np.float32)
    n = x.shape[-1]
    y = np.empty_like(x)
    lib().gdn2o_rmsnorm_gate(_ptr(x), _ptr(gate), _ptr(weight), x.size // n, n, float(eps), _ptr(y))
    return y


# ---------------------------------------------------------------------------
# Layer (src/module.rs, src/config.rs)
# ---------------------------------------------------------------------------
class _Cfg(ctypes.Structure):
    _fields_ = [
        ("hidden", ctypes.c_int), ("heads", ctypes.c_int), ("head_dim", ctypes.c_int),
        ("num_v_heads", ctypes.c_int), ("head_v_dim", ctypes.c_int),
        ("use_short_conv", ctypes.c_int), ("allow_neg_eigval", ctypes.c_int),
        ("mode_chunk", ctypes.c_int), ("chunk_size", ctypes.c_int), ("has_min_decay", ctypes.c_int),
        ("min_decay", ctypes.c_double), ("norm_eps", ctypes.c_double), ("gva_scrambled", ctypes.c_int),
    ]


WEIGHT_NAMES = ("q_proj", "k_proj", "v_proj", "f_proj_0", "f_proj_1", "b_proj", "w_proj", "g_proj_0",
                "g_proj_1", "g_proj_1_bias", "a_log", "dt_bias", "o_norm_weight", "o_proj", "q_conv_w",
                "k_conv_w", "v_conv_w", "decay_factors")


class _W(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in WEIGHT_NAMES]


@dataclass
class OracleState:
    """Gdn2State (src/module.rs:30-63) in double: recurrent [B,HV,K,V], conv caches [B,3,kd|vd]."""
    recurrent: np.ndarray
    conv_q: np.ndarray
    conv_k: np.ndarray
    conv_v: np.ndarray


@dataclass
class LayerResult:
    out: np.ndarray
    o_core: np.ndarray
    proj: dict = field(default_factory=dict)


def layer_forward(cfg, weights: dict, x, state: Optional[OracleState] = None, gva_scrambled=False,
                  want_proj=False):
    """GatedDeltaNet2::forward(x, &mut state, true) / forward_train(x) in double.

    cfg: object with hidden_size, num_heads, head_dim, expand_v, num_v_heads,
    use_short_conv, allow_neg_eigval, norm_eps, chunk_size, min_decay.
    state None = Option::None on entry (forward_train is the same call with
    the returned state discarded).  Returns (LayerResult, new OracleState).
    """
    H, K = cfg.num_heads, cfg.head_dim
    HV = cfg.num_v_heads or H
    V = int(K * cfg.expand_v)
    kd, vd = H * K, HV * V
    x = _c(x, np.float32)
    B, T, D = x.shape
    c = _Cfg(D, H, K, HV, V, int(cfg.use_short_conv), int(cfg.allow_neg_eigval), 1, int(cfg.chunk_size),
             int(cfg.min_decay is not None), float(cfg.min_decay or 0.0), float(cfg.norm_eps),
             int(gva_scrambled))
    keep = {n: (None if weights.get(n) is None else _c(weights[n], np.float32)) for n in WEIGHT_NAMES}
    wst = _W(**{n: (None if a is None else a.ctypes.data) for n, a in keep.items()})
    if state is None:
        S = np.zeros((B, HV, K, V), np.float64)
        cq = np.zeros((B, 3, kd), np.float64)
        ck = np.zeros((B, 3, kd), np.float64)
        cv = np.zeros((B, 3, vd), np.float64)
        has = 0
    else:
        S = np.array(state.recurrent, np.float64, order="C", copy=True)
        cq = np.array(state.conv_q, np.float64, order="C", copy=True)
        ck = np.array(state.conv_k, np.float64, order="C", copy=True)
        cv = np.array(state.conv_v, np.float64, order="C", copy=True)
        has = 1
    out = np.empty((B, T, D), np.float64)
    oc = np.empty((B, HV, T, V), np.float64)
    Hk = HV if (gva_scrambled and HV > H) else H
    proj = {}
    if want_proj:
        proj = {n: np.empty((B, Hk, T, K), np.float64) for n in ("q", "k", "g", "b")}
        proj.update({n: np.empty((B, HV, T, V), np.float64) for n in ("v", "w")})
        proj["gate"] = np.empty((B, T, HV, V), np.float64)
    pp = [_ptr(proj.get(n)) for n in ("q", "k", "g", "b", "v", "w", "gate")]
    lib().gdn2o_layer_forward(ctypes.byref(c), ctypes.byref(wst), _ptr(x), B, T, has, _ptr(S), _ptr(cq),
                              _ptr(ck), _ptr(cv), _ptr(out), _ptr(oc), *pp)
    if not cfg.use_short_conv and state is not None:
        cq, ck, cv = state.conv_q, state.conv_k, state.conv_v
    return LayerResult(out, oc, proj), OracleState(S, cq, ck, cv)


def _cfg_struct(cfg, gva_scrambled):
    H, K = cfg.num_heads, cfg.head_dim
    HV = cfg.num_v_heads or H
    V = int(K * cfg.expand_v)
    return _Cfg(cfg.hidden_size, H, K, HV, V, int(cfg.use_short_conv), int(cfg.allow_neg_eigval), 1,
                int(cfg.chunk_size), int(cfg.min_decay is not None), float(cfg.min_decay or 0.0),
                float(cfg.norm_eps), int(gva_scrambled)), H, K, HV, V


RAW_NAMES = ("q_raw", "k_raw", "f_raw", "b_raw", "v_raw", "w_raw", "gate")


def layer_from_raw(cfg, weights: dict, raw: dict, state: Optional[OracleState] = None, gva_scrambled=False):
    """The layer after its Linear layers (src/module.rs:404-476, :244-312), in double.

    raw: Linear outputs [B, T, n]: q_raw, k_raw, f_raw, b_raw (n = kd) and
    v_raw, w_raw, gate (n = vd, gate with the g_proj_1 bias).  Returns
    (o_norm [B, T, vd] = input of o_proj, o_core [B, HV, T, V], new state).
    """
    c, H, K, HV, V = _cfg_struct(cfg, gva_scrambled)
    kd, vd = H * K, HV * V
    rr = {n: _c(raw[n], np.float64) for n in RAW_NAMES}
    B, T = rr["q_raw"].shape[:2]
    keep = {n: (None if weights.get(n) is None else _c(weights[n], np.float32)) for n in WEIGHT_NAMES}
    wst = _W(**{n: (None if a is None else a.ctypes.data) for n, a in keep.items()})
    if state is None:
        S = np.zeros((B, HV, K, V), np.float64)
        cq, ck, cv = (np.zeros((B, 3, n), np.float64) for n in (kd, kd, vd))
        has = 0
    else:
        S = np.array(state.recurrent, np.float64, order="C", copy=True)
        cq = np.array(state.conv_q, np.float64, order="C", copy=True)
        ck = np.array(state.conv_k, np.float64, order="C", copy=True)
        cv = np.array(state.conv_v, np.float64, order="C", copy=True)
        has = 1
    on = np.empty((B, T, vd), np.float64)
    oc = np.empty((B, HV, T, V), np.float64)
    lib().gdn2o_layer_from_raw(ctypes.byref(c), ctypes.byref(wst), *(_ptr(rr[n]) for n in RAW_NAMES), B, T, has,
                               _ptr(S), _ptr(cq), _ptr(ck), _ptr(cv), _ptr(on), _ptr(oc),
                               None, None, None, None, None, None)
    return on, oc, OracleState(S, cq, ck, cv)


def layer_forward_f32_host(cfg, weights: dict, x):
    """forward_train(x) from a zero state the way the reference's CPU backend
    computes it, as f32 tensor operations: Linear layers through BLAS sgemm
    (numpy), short conv as four shifted multiply-adds over the replicate-padded
    input (src/short_conv.rs:22-65), the gates (src/module.rs:417-443), L2
    norm (src/l2norm.rs:13-16), the f32 chunk_wy_forward restatement
    (src/forward.rs:44-278) and gated RMSNorm (src/module.rs:501-517).  Used as
    bench.py's full-layer CPU baseline; tests/test_oracle.py checks it against
    layer_forward.  Short conv on; GVA, neg-eig and min_decay are not covered.
    Returns out [B, T, D] (float32)."""
    H, K = cfg.num_heads, cfg.head_dim
    HV = cfg.num_v_heads or H
    V = int(K * cfg.expand_v)
    if HV != H or cfg.allow_neg_eigval or cfg.min_decay is not None or not cfg.use_short_conv:
        raise ValueError("layer_forward_f32_host: short conv on, HV == H, no neg-eig, no min_decay only")
    kd, vd = H * K, HV * V
    W = {n: (None if a is None else np.asarray(a, np.float32)) for n, a in weights.items()}
    x = _c(x, np.float32)
    B, T, D = x.shape
    x2 = x.reshape(B * T, D)

    def silu(a):
        return a / (np.float32(1) + np.exp(-a))

    def conv(n_proj, n_w, n):
        y = (x2 @ W[n_proj]).reshape(B, T, n)
        pad = np.concatenate([np.repeat(y[:, :1], 3, axis=1), y], axis=1)
        wc = W[n_w]
        acc = pad[:, 0:T] * wc[:, 0]
        for i in range(1, 4):
            acc += pad[:, i:i + T] * wc[:, i]
        return silu(acc)

    def heads(a, n):  # [B, T, H * n] -> [B, H, T, n]
        return np.ascontiguousarray(a.reshape(B, T, -1, n).transpose(0, 2, 1, 3), dtype=np.float32)

    def l2n(a):
        return a / np.sqrt(np.sum(a * a, axis=-1, keepdims=True) + np.float32(1e-6))

    q = l2n(heads(conv("q_proj", "q_conv_w", kd), K))
    k = l2n(heads(conv("k_proj", "k_conv_w", kd), K))
    v = heads(conv("v_proj", "v_conv_w", vd), V)
    f = ((x2 @ W["f_proj_0"]) @ W["f_proj_1"]).reshape(B, T, H, K) + W["dt_bias"].reshape(H, K)
    g = -np.exp(W["a_log"])[:, None] * np.logaddexp(np.float32(0), f)
    b = np.float32(1) / (np.float32(1) + np.exp(-(x2 @ W["b_proj"])))
    w = np.float32(1) / (np.float32(1) + np.exp(-(x2 @ W["w_proj"])))
    gate = ((x2 @ W["g_proj_0"]) @ W["g_proj_1"] + W["g_proj_1_bias"]).reshape(B, T, HV, V)
    o, _ = chunk_wy_f32(q, k, v, heads(g.reshape(B, T, kd), K), heads(b, K), heads(w, V), scale=K ** -0.5,
                        chunk_size=cfg.chunk_size)
    o = o.transpose(0, 2, 1, 3)  # [B, T, HV, V]
    y = o / np.sqrt(np.mean(o * o, axis=-1, keepdims=True) + np.float32(cfg.norm_eps)) * W["o_norm_weight"] * silu(gate)
    return (y.reshape(B * T, vd) @ W["o_proj"]).reshape(B, T, D).astype(np.float32)


# ---------------------------------------------------------------------------
# Layer adjoint (the gradients burn's autodiff takes through forward /
# forward_train, tests/autodiff.rs:153-205), in double.
# ---------------------------------------------------------------------------
def _sig(x):
    return 1.0 / (1.0 + np.exp(-x))


def _silu(x):
    return x * _sig(x)


def _dsilu(x):
    s = _sig(x)
    return s * (1.0 + x * (1.0 - s))


def _softplus(x):
    """ln(1 + e^x), evaluated without overflow (burn's softplus with beta = 1)."""
    return np.maximum(x, 0.0) + np.log1p(np.exp(-np.abs(x)))


def scan_d(q, k, v, g, b, w, S0, scale):
    """The per-token scan on double operands (q, k, g, b [B,H,T,K] with true
    head repeat for GVA).  Returns (out [B,HV,T,V], S_T)."""
    q, k, v, g, b, w = (_c(a, np.float64) for a in (q, k, v, g, b, w))
    B, Hk, T, K = q.shape
    HV, V = v.shape[1], v.shape[3]
    S = np.array(S0, np.float64, order="C", copy=True)
    out = np.empty((B, HV, T, V), np.float64)
    lib().gdn2o_scan_d(*(_ptr(a) for a in (q, k, v, g, b, w, S)), B, HV, Hk, T, K, V, float(scale), _ptr(out))
    return out, S


def recurrent_bwd_d(q, k, v, g, b, w, d_out, S0=None, d_ST=None, scale=1.0):
    """recurrent_bwd_f64 on double operands (full-width g and b)."""
    q, k, v, g, b, w = (_c(a, np.float64) for a in (q, k, v, g, b, w))
    B, Hk, T, K = q.shape
    HV, V = v.shape[1], v.shape[3]
    S0 = None if S0 is None else _c(S0, np.float64)
    d_out = _c(d_out, np.float64)
    d_ST = None if d_ST is None else _c(d_ST, np.float64)
    r = {"dq": np.empty(q.shape), "dk": np.empty(k.shape), "dg": np.empty(g.shape), "db": np.empty(b.shape),
         "dv": np.empty(v.shape), "dw": np.empty(w.shape), "dS0": np.empty((B, HV, K, V))}
    lib().gdn2o_recurrent_bwd_d(*(_ptr(a) for a in (q, k, v, g, b, w, S0, d_out, d_ST)), B, HV, Hk, T, K, V, K, K,
                                float(scale), *(_ptr(r[n]) for n in ("dq", "dk", "dg", "db", "dv", "dw", "dS0")))
    return r


@dataclass
class LayerGrads:
    out: np.ndarray          # the forward's output [B, T, D] (recomputed)
    dx: np.ndarray           # [B, T, D]
    params: dict             # parameter name -> gradient (None for an absent parameter)
    d_state: OracleState     # gradient of the state on entry (zeros for the conv caches of Option::None)


def layer_backward_f64(cfg, weights: dict, x, d_out, state: Optional[OracleState] = None,
                       d_state: Optional[OracleState] = None, gva_scrambled=False) -> LayerGrads:
    """Gradients of L = <d_out, out> + <d_state, state after the call> for
    GatedDeltaNet2::forward(x, &mut state, true) (src/module.rs:224-316;
    state None = Option::None, which is forward_train, :326-375), true head
    repeat for GVA.  Everything is recomputed from x in double: Linear layers
    (y = x W), short conv with replicate padding or cache
    (src/short_conv.rs:22-65), gates (src/module.rs:417-443), L2 norm
    (src/l2norm.rs:13-16), the scan (gdn2o_scan_d / gdn2o_recurrent_bwd_d)
    and the gated RMSNorm (src/module.rs:501-517).  Without short conv the
    conv caches pass through unchanged, so their gradient passes through.
    gva_scrambled: the reference's GVA layout (src/module.rs:456-468,
    unsqueeze at 3, repeat, reshape to [B, HV, T, K]) instead of head repeat;
    its adjoint sums each key element's rep copies."""
    H, K = cfg.num_heads, cfg.head_dim
    HV = cfg.num_v_heads or H
    V = int(K * cfg.expand_v)
    kd, vd = H * K, HV * V
    sc, neg, md = bool(cfg.use_short_conv), bool(cfg.allow_neg_eigval), cfg.min_decay
    W = {n: (None if weights.get(n) is None else np.asarray(weights[n], np.float64)) for n in WEIGHT_NAMES}
    x = np.asarray(x, np.float64)
    B, T, D = x.shape
    M = B * T
    X = x.reshape(M, D)
    dY = np.asarray(d_out, np.float64).reshape(M, D)
    names = {"q": "q_proj", "k": "k_proj", "v": "v_proj", "b": "b_proj", "w": "w_proj"}
    raw = {n: X @ W[p] for n, p in names.items()}
    f0 = X @ W["f_proj_0"]
    f_raw = f0 @ W["f_proj_1"]
    g0 = X @ W["g_proj_0"]
    gate = g0 @ W["g_proj_1"] + W["g_proj_1_bias"]
    width = {"q": kd, "k": kd, "v": vd}
    caches = None if state is None else {"q": state.conv_q, "k": state.conv_k, "v": state.conv_v}
    xpad, u = {}, {}
    for n, C in width.items():
        r = raw[n].reshape(B, T, C)
        if sc:
            pad = np.repeat(r[:, :1], 3, axis=1) if caches is None else np.asarray(caches[n], np.float64)
            xp = np.concatenate([pad, r], axis=1)
            wc = W[n + "_conv_w"]
            u[n] = sum(xp[:, i:i + T] * wc[:, i] for i in range(4))
            xpad[n] = xp
        else:
            u[n] = r
    A = np.repeat(np.exp(W["a_log"]), K)
    xg = f_raw + W["dt_bias"]
    g_pre = -A * _softplus(xg)
    if md is not None:
        sdf = _sig(W["decay_factors"].reshape(kd))
        e = sdf * (1.0 - md) * np.exp(g_pre)
        gg = np.log(e + md)
    else:
        gg = g_pre
    bs, ws = _sig(raw["b"]), _sig(raw["w"])
    bmul = 2.0 if neg else 1.0
    qa = _silu(u["q"]).reshape(B, T, H, K)
    ka = _silu(u["k"]).reshape(B, T, H, K)
    nq = np.sqrt((qa * qa).sum(-1, keepdims=True) + 1e-6)
    nk = np.sqrt((ka * ka).sum(-1, keepdims=True) + 1e-6)
    qn, kn = qa / nq, ka / nk

    def to4(a, n, d):
        return np.ascontiguousarray(a.reshape(B, T, n, d).transpose(0, 2, 1, 3))

    def back(a):
        return a.transpose(0, 2, 1, 3).reshape(M, -1)

    q4, k4, g4, b4 = to4(qn, H, K), to4(kn, H, K), to4(gg, H, K), to4(bs * bmul, H, K)
    v4, w4 = to4(_silu(u["v"]), HV, V), to4(ws, HV, V)
    rep = HV // H
    scr = gva_scrambled and rep > 1
    if scr:  # [B, H, T, K] -> [B, H, T, rep, K] -> [B, HV, T, K] (src/module.rs:459-463)
        q4, k4, g4, b4 = (np.repeat(a[:, :, :, None, :], rep, axis=3).reshape(B, HV, T, K)
                          for a in (q4, k4, g4, b4))
    S0 = np.zeros((B, HV, K, V)) if state is None else np.asarray(state.recurrent, np.float64)
    scale = float(K) ** -0.5
    O, _ = scan_d(q4, k4, v4, g4, b4, w4, S0, scale)
    Ob = O.transpose(0, 2, 1, 3)
    G4 = gate.reshape(B, T, HV, V)
    rms = np.sqrt((Ob * Ob).mean(-1, keepdims=True) + cfg.norm_eps)
    nrm, z, wn = Ob / rms, _silu(G4), W["o_norm_weight"]
    y = (nrm * wn * z).reshape(M, vd)
    out = (y @ W["o_proj"]).reshape(B, T, D)

    g = {}
    g["o_proj"] = y.T @ dY
    dy = (dY @ W["o_proj"].T).reshape(B, T, HV, V)
    dn = dy * wn * z
    g["o_norm_weight"] = (dy * nrm * z).reshape(-1, V).sum(0)
    dgate = (dy * nrm * wn * _dsilu(G4)).reshape(M, vd)
    dOb = (dn - nrm * (dn * nrm).mean(-1, keepdims=True)) / rms
    r = recurrent_bwd_d(q4, k4, v4, g4, b4, w4, dOb.transpose(0, 2, 1, 3), S0,
                        None if d_state is None else d_state.recurrent, scale)
    if scr:  # adjoint of the repeat + reshape: each key element's rep copies summed
        for n in ("dq", "dk", "dg", "db"):
            r[n] = r[n].reshape(B, H, T, rep, K).sum(3)
    dqn, dkn = back(r["dq"]).reshape(B, T, H, K), back(r["dk"]).reshape(B, T, H, K)
    dqa = (dqn - qn * (dqn * qn).sum(-1, keepdims=True)) / nq
    dka = (dkn - kn * (dkn * kn).sum(-1, keepdims=True)) / nk
    dgg, dbb, dva, dws = back(r["dg"]), back(r["db"]), back(r["dv"]), back(r["dw"])
    if md is not None:
        dg_pre = dgg * e / (e + md)
        g["decay_factors"] = ((dgg * np.exp(g_pre) * (1.0 - md) * sdf * (1.0 - sdf) / (e + md)).sum(0)
                              .reshape(np.shape(W["decay_factors"])))
    else:
        dg_pre = dgg
        g["decay_factors"] = None
    g["a_log"] = (dg_pre * g_pre).sum(0).reshape(H, K).sum(1)
    dxg = dg_pre * (-A) * _sig(xg)
    g["dt_bias"] = dxg.sum(0)
    draw = {"b": dbb * bmul * bs * (1.0 - bs), "w": dws * ws * (1.0 - ws)}
    du = {"q": dqa.reshape(B, T, kd) * _dsilu(u["q"]), "k": dka.reshape(B, T, kd) * _dsilu(u["k"]),
          "v": dva.reshape(B, T, vd) * _dsilu(u["v"])}
    dconv = {}
    for n, C in width.items():
        d_out_cache = None if d_state is None else np.asarray(getattr(d_state, "conv_" + n), np.float64)
        if sc:
            wc = W[n + "_conv_w"]
            dxp = np.zeros((B, T + 3, C))
            for i in range(4):
                dxp[:, i:i + T] += du[n] * wc[:, i]
            if d_out_cache is not None:
                dxp[:, T:T + 3] += d_out_cache
            g[n + "_conv_w"] = np.stack([(du[n] * xpad[n][:, i:i + T]).sum((0, 1)) for i in range(4)], axis=1)
            dr = dxp[:, 3:].copy()
            if caches is None:
                dr[:, 0] += dxp[:, :3].sum(1)
                dconv[n] = np.zeros((B, 3, C))
            else:
                dconv[n] = dxp[:, :3].copy()
        else:
            dr = du[n]
            g[n + "_conv_w"] = np.zeros((C, 4))
            dconv[n] = (d_out_cache.copy() if (d_out_cache is not None and state is not None)
                        else np.zeros((B, 3, C)))
        draw[n] = dr.reshape(M, C)
    dX = np.zeros((M, D))
    for n, p in names.items():
        g[p] = X.T @ draw[n]
        dX += draw[n] @ W[p].T
    g["f_proj_1"] = f0.T @ dxg
    df0 = dxg @ W["f_proj_1"].T
    g["f_proj_0"] = X.T @ df0
    dX += df0 @ W["f_proj_0"].T
    g["g_proj_1"] = g0.T @ dgate
    g["g_proj_1_bias"] = dgate.sum(0)
    dg0 = dgate @ W["g_proj_1"].T
    g["g_proj_0"] = X.T @ dg0
    dX += dg0 @ W["g_proj_0"].T
    return LayerGrads(out, dX.reshape(B, T, D), g, OracleState(r["dS0"], dconv["q"], dconv["k"], dconv["v"]))

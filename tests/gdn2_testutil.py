"""Test helpers: a config record and seeded weights drawn from the
reference's initialisers (src/module.rs:121-187), in burn's [in, out]
Linear layout.  Both the oracle and the GPU path consume the same arrays."""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import numpy as np


@dataclass
class Cfg:
    """Field names of Gdn2Config (src/config.rs:23-58)."""
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

    @property
    def hv(self):
        return self.num_v_heads or self.num_heads

    @property
    def v_head(self):
        return int(self.head_dim * self.expand_v)

    @property
    def kd(self):
        return self.num_heads * self.head_dim

    @property
    def vd(self):
        return self.hv * self.v_head


def init_weights(cfg: Cfg, seed: int = 1337, dt_bias_shift: float = 0.0) -> dict:
    rng = np.random.default_rng(seed)
    D, H, K, kd, vd, V = cfg.hidden_size, cfg.num_heads, cfg.head_dim, cfg.kd, cfg.vd, cfg.v_head
    gain = 2.0 ** -2.5

    def lin(i, o):
        bound = gain * math.sqrt(6.0 / (i + o))
        return rng.uniform(-bound, bound, (i, o)).astype(np.float32)

    W = {
        "q_proj": lin(D, kd), "k_proj": lin(D, kd), "v_proj": lin(D, vd),
        "f_proj_0": lin(D, V), "f_proj_1": lin(V, kd),
        "b_proj": lin(D, kd), "w_proj": lin(D, vd),
        "g_proj_0": lin(D, V), "g_proj_1": lin(V, vd),
        "g_proj_1_bias": np.zeros(vd, np.float32),
        "o_proj": lin(vd, D),
        "q_conv_w": rng.uniform(-0.5, 0.5, (kd, 4)).astype(np.float32),
        "k_conv_w": rng.uniform(-0.5, 0.5, (kd, 4)).astype(np.float32),
        "v_conv_w": rng.uniform(-0.5, 0.5, (vd, 4)).astype(np.float32),
        "a_log": rng.uniform(math.log(1.0), math.log(16.0), H).astype(np.float32),
        "o_norm_weight": np.ones(V, np.float32),
    }
    dt = np.maximum(np.exp(rng.uniform(math.log(1e-3), math.log(0.1), kd)), 1e-4)
    W["dt_bias"] = (dt + np.log(-np.expm1(-dt)) + dt_bias_shift).astype(np.float32)
    W["decay_factors"] = np.full(H * K, 2.0, np.float32) if cfg.min_decay is not None else None
    return W


def maxabs(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))

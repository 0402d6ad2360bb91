"""Pins the oracle's layer adjoint (oracle.layer_backward_f64) against
central finite differences of the oracle's layer forward (gdn2o_layer_forward,
a separate C implementation pinned by the reference's golden vectors in
test_oracle.py): every parameter, the input and every part of the state, on
configurations with and without short conv, with GVA (head repeat and the
reference's layout), negative eigenvalues, min_decay, a carried state, fewer
than three tokens and a single token.
The loss is L = <d_out, out> + <d_state, state after the call>.  CPU only."""
import copy

import numpy as np
import pytest

from gdn2_testutil import Cfg, init_weights
from oracle import oracle as O


def _loss(cfg, W, x, state, d_out, d_state, scrambled=False):
    st = None if state is None else copy.deepcopy(state)
    res, new = O.layer_forward(cfg, W, x, st, gva_scrambled=scrambled)
    L = float((res.out * d_out).sum())
    if d_state is not None:
        for f in ("recurrent", "conv_q", "conv_k", "conv_v"):
            L += float((np.asarray(getattr(new, f)) * getattr(d_state, f)).sum())
    return L, res.out


def _rand_state(rng, B, cfg):
    K, V, kd, vd = cfg.head_dim, cfg.v_head, cfg.kd, cfg.vd
    return O.OracleState(rng.normal(0, 0.5, (B, cfg.hv, K, V)), rng.normal(0, 1.0, (B, 3, kd)),
                         rng.normal(0, 1.0, (B, 3, kd)), rng.normal(0, 1.0, (B, 3, vd)))


CASES = [
    # id, cfg kwargs, B, T, carried state, d_state
    ("conv", dict(hidden_size=8, num_heads=2, head_dim=4), 2, 5, False, False),
    ("gva_neg_mindecay_state_T2", dict(hidden_size=8, num_heads=1, head_dim=4, num_v_heads=2, expand_v=1.5,
                                       allow_neg_eigval=True, min_decay=0.9), 2, 2, True, True),
    ("noconv_state", dict(hidden_size=6, num_heads=2, head_dim=3, use_short_conv=False), 1, 6, True, True),
    ("conv_T1", dict(hidden_size=8, num_heads=2, head_dim=4), 2, 1, False, True),
    # the reference's GVA layout (value head h rep + a at time t reads key time (a T + t) / rep)
    ("gva_reference_layout_state", dict(hidden_size=8, num_heads=1, head_dim=4, num_v_heads=3,
                                        allow_neg_eigval=True), 2, 5, True, True, True),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_layer_adjoint_matches_finite_differences(case):
    _, kw, B, T, carried, with_ds = case[:6]
    scr = len(case) > 6 and case[6]
    cfg = Cfg(**kw)
    rng = np.random.default_rng(7)
    W = init_weights(cfg, seed=11)
    # non-trivial values where the initialisers give constants
    W["o_norm_weight"] = rng.uniform(0.5, 1.5, W["o_norm_weight"].shape).astype(np.float32)
    W["g_proj_1_bias"] = rng.normal(0, 0.3, W["g_proj_1_bias"].shape).astype(np.float32)
    if W["decay_factors"] is not None:
        W["decay_factors"] = rng.normal(0, 1.0, W["decay_factors"].shape).astype(np.float32)
    for n in ("q_proj", "k_proj", "v_proj", "b_proj", "w_proj", "f_proj_0", "g_proj_0", "o_proj"):
        W[n] = (W[n] * 8).astype(np.float32)  # O(1) activations so every nonlinearity is exercised
    x = rng.normal(0, 1, (B, T, cfg.hidden_size)).astype(np.float32)
    state = _rand_state(rng, B, cfg) if carried else None
    d_out = rng.normal(0, 1, (B, T, cfg.hidden_size))
    d_state = _rand_state(rng, B, cfg) if with_ds else None

    G = O.layer_backward_f64(cfg, W, x, d_out, state, d_state, gva_scrambled=scr)
    _, out = _loss(cfg, W, x, state, d_out, d_state, scr)
    assert np.max(np.abs(G.out - out)) <= 1e-12 * max(1.0, np.max(np.abs(out)))

    worst = 0.0

    def check(name, an, fd):
        nonlocal worst
        err = abs(fd - an) / max(1e-3, abs(an))
        worst = max(worst, err)
        assert abs(fd - an) <= 1e-6 + 1e-5 * abs(an), (name, fd, an)

    # float32 inputs: step between the two neighbouring float32 values actually fed
    f32_inputs = [("x", x, G.dx)] + [(n, W[n], G.params[n]) for n in O.WEIGHT_NAMES if W.get(n) is not None]
    for name, arr, grad in f32_inputs:
        if name.endswith("_conv_w") and not cfg.use_short_conv:
            assert np.all(grad == 0)
            continue
        flat, gflat = arr.reshape(-1), np.asarray(grad).reshape(-1)
        assert gflat.size == flat.size, name
        for e in rng.choice(flat.size, size=min(5, flat.size), replace=False):
            x0 = flat[e]
            h = np.float32(2.0 ** -14) * max(np.float32(1.0), abs(x0))
            xp, xm = np.float32(x0 + h), np.float32(x0 - h)
            flat[e] = xp
            lp, _ = _loss(cfg, W, x, state, d_out, d_state, scr)
            flat[e] = xm
            lm, _ = _loss(cfg, W, x, state, d_out, d_state, scr)
            flat[e] = x0
            check(name, gflat[e], (lp - lm) / (float(xp) - float(xm)))
    # double state entries
    if state is not None:
        for f in ("recurrent", "conv_q", "conv_k", "conv_v"):
            flat, gflat = getattr(state, f).reshape(-1), getattr(G.d_state, f).reshape(-1)
            for e in rng.choice(flat.size, size=min(5, flat.size), replace=False):
                x0 = flat[e]
                flat[e] = x0 + 1e-5
                lp, _ = _loss(cfg, W, x, state, d_out, d_state, scr)
                flat[e] = x0 - 1e-5
                lm, _ = _loss(cfg, W, x, state, d_out, d_state, scr)
                flat[e] = x0
                check(f, gflat[e], (lp - lm) / 2e-5)
    else:
        for f in ("conv_q", "conv_k", "conv_v"):
            assert np.all(getattr(G.d_state, f) == 0)
    print(f"worst relative FD error {worst:.2e}")

"""Pins the oracle's adjoint of the recurrence (gdn2o_recurrent_bwd_f64)
against central finite differences of the oracle's forward (itself pinned in
test_oracle.py) and against the linear-attention closed form.  CPU only."""
import numpy as np
import pytest

from conftest import rand_inputs
from oracle import oracle as O


def _loss(ins, S0, d_out, d_ST, scale):
    out, S = O.recurrent_f64(*ins, S0=S0, scale=scale)
    return float((out * d_out).sum() + (S * d_ST).sum())


def _fd_check(ins, S0, d_out, d_ST, scale, grads, rng, per_tensor=12):
    """Central differences on a random sample of elements of every input.
    q, k, g, b, v, w are float32 inputs: the step is taken between the two
    neighbouring float32 values actually fed to the forward."""
    names = ("q", "k", "v", "g", "b", "w")
    worst = 0.0
    for ti, name in enumerate(names):
        x = ins[ti]
        flat = x.reshape(-1)
        for e in rng.choice(flat.size, size=min(per_tensor, flat.size), replace=False):
            x0 = flat[e]
            h = np.float32(2.0 ** -9) * max(np.float32(1.0), abs(x0))
            xp, xm = np.float32(x0 + h), np.float32(x0 - h)
            flat[e] = xp
            lp = _loss(ins, S0, d_out, d_ST, scale)
            flat[e] = xm
            lm = _loss(ins, S0, d_out, d_ST, scale)
            flat[e] = x0
            fd = (lp - lm) / (float(xp) - float(xm))
            an = grads["d" + name].reshape(-1)[e]
            err = abs(fd - an) / max(1.0, abs(an))
            worst = max(worst, err)
            assert err < 2e-5, (name, e, fd, an)
    # S0 is a double input: plain central differences
    flat = S0.reshape(-1)
    for e in rng.choice(flat.size, size=per_tensor, replace=False):
        x0 = flat[e]
        flat[e] = x0 + 1e-4
        lp = _loss(ins, S0, d_out, d_ST, scale)
        flat[e] = x0 - 1e-4
        lm = _loss(ins, S0, d_out, d_ST, scale)
        flat[e] = x0
        fd = (lp - lm) / 2e-4
        an = grads["dS0"].reshape(-1)[e]
        assert abs(fd - an) / max(1.0, abs(an)) < 2e-6, ("S0", e, fd, an)
    return worst


CASES = [
    # B, Hk, HV, T, K, V, g range, b_hi, gdim, bdim
    (1, 1, 1, 6, 4, 3, (-0.3, -0.02), 1.0, None, None),
    (2, 1, 2, 9, 5, 4, (-1.5, -0.2), 2.0, None, None),  # GVA rep 2, negative eigenvalues
    (1, 2, 2, 7, 4, 6, (-0.5, -0.05), 1.0, 1, 1),       # scalar-broadcast g and b
]


@pytest.mark.parametrize("case", CASES, ids=["plain", "gva_negeig", "broadcast_gb"])
def test_recurrent_bwd_matches_finite_differences(case):
    B, Hk, HV, T, K, V, (glo, ghi), bhi, gdim, bdim = case
    rng = np.random.default_rng(31 + T)
    q, k, v, g, b, w = rand_inputs(rng, B, Hk, HV, T, K, V, g_lo=glo, g_hi=ghi, b_hi=bhi, gdim=gdim, bdim=bdim)
    S0 = rng.standard_normal((B, HV, K, V)) * 0.5
    d_out = rng.standard_normal((B, HV, T, V))
    d_ST = rng.standard_normal((B, HV, K, V))
    ins = [q, k, v, g, b, w]
    grads = O.recurrent_bwd_f64(*ins, d_out, S0=S0, d_ST=d_ST, scale=0.6)
    assert grads["dg"].shape == g.shape and grads["db"].shape == b.shape and grads["dq"].shape == q.shape
    _fd_check(ins, S0, d_out, d_ST, 0.6, grads, rng)


def test_recurrent_bwd_linear_attention_closed_form():
    """b = 0, g = 0: out_t = scale sum_{s<=t} (q_t . k_s) u_s with u = w v, and
    S_T = S0 + sum_s k_s u_s^T; the gradients of q, k, v, w, S0 in closed form."""
    rng = np.random.default_rng(3)
    B, H, T, K, V = 1, 2, 11, 6, 5
    q, k, v, g, b, w = rand_inputs(rng, B, H, H, T, K, V)
    g[:] = 0
    b[:] = 0
    S0 = rng.standard_normal((B, H, K, V))
    dO = rng.standard_normal((B, H, T, V))
    dST = rng.standard_normal((B, H, K, V))
    sc = 0.8
    r = O.recurrent_bwd_f64(q, k, v, g, b, w, dO, S0=S0, d_ST=dST, scale=sc)
    q64, k64, u = q.astype(np.float64), k.astype(np.float64), w.astype(np.float64) * v
    M = np.tril(np.ones((T, T)))                                      # M[t, s] = s <= t
    P = np.einsum("bhtv,bhsv->bhts", dO, u) * M                        # dO_t . u_s
    A = np.einsum("bhtk,bhsk->bhts", q64, k64) * M                     # q_t . k_s
    dq = sc * (np.einsum("bhts,bhsk->bhtk", P, k64) + np.einsum("bhkv,bhtv->bhtk", S0, dO))
    dk = sc * np.einsum("bhts,bhtk->bhsk", P, q64) + np.einsum("bhkv,bhsv->bhsk", dST, u)
    du = sc * np.einsum("bhts,bhtv->bhsv", A, dO) + np.einsum("bhkv,bhsk->bhsv", dST, k64)
    dS0 = sc * np.einsum("bhtk,bhtv->bhkv", q64, dO) + dST
    assert np.abs(r["dq"] - dq).max() < 1e-10
    assert np.abs(r["dk"] - dk).max() < 1e-10
    assert np.abs(r["dv"] - du * w).max() < 1e-10
    assert np.abs(r["dw"] - du * v).max() < 1e-10
    assert np.abs(r["dS0"] - dS0).max() < 1e-10

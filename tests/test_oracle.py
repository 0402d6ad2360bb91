"""Pins the CPU oracle (oracle/gdn2_oracle.c) against things other than
itself: closed forms, algebraic identities of the delta rule, brute force
on tiny inputs, the reference's own invariants and the golden vectors of
the reference's torch model.  CPU only."""
import os

import numpy as np
import pytest

from conftest import rand_inputs
from gdn2_testutil import Cfg, init_weights, maxabs
from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "layer_d64_h4.npz")


# --------------------------------------------------------------------------
# recurrence (src/kernel/fused_recurrent.rs:27-52)
# --------------------------------------------------------------------------
def test_recurrence_linear_attention_closed_form():
    """b = 0, g = 0: S_T = sum_t k_t (w_t v_t)^T and
    o_t = scale * sum_{s<=t} (q_t . k_s) w_s v_s (plain linear attention)."""
    rng = np.random.default_rng(1)
    q, k, v, g, b, w = rand_inputs(rng, 2, 3, 3, 17, 8, 5)
    g[:] = 0
    b[:] = 0
    out, S = O.recurrent_f64(q, k, v, g, b, w, scale=0.7)
    wv = (w.astype(np.float64) * v)
    S_ref = np.einsum("bhtk,bhtv->bhkv", k.astype(np.float64), wv)
    A = np.einsum("bhtk,bhsk->bhts", q.astype(np.float64), k.astype(np.float64))
    A = np.tril(A)
    o_ref = 0.7 * np.einsum("bhts,bhsv->bhtv", A, wv)
    assert maxabs(S, S_ref) < 1e-12
    assert maxabs(out, o_ref) < 1e-12


def test_recurrence_gated_linear_attention_closed_form():
    """b = 0: o_t = scale * sum_{s<=t} sum_c q_t k_s exp(G_t - G_s) w_s v_s with
    G the per-channel cumulative log decay (gated linear attention)."""
    rng = np.random.default_rng(2)
    q, k, v, g, b, w = rand_inputs(rng, 1, 2, 2, 13, 6, 4, g_lo=-1.0, g_hi=-0.01)
    b[:] = 0
    S0 = rng.standard_normal((1, 2, 6, 4))
    out, S = O.recurrent_f64(q, k, v, g, b, w, S0=S0, scale=1.0)
    G = np.cumsum(g.astype(np.float64), axis=2)
    wv = w.astype(np.float64) * v
    qd, kd = q.astype(np.float64), k.astype(np.float64)
    T = q.shape[2]
    o_ref = np.zeros_like(out)
    for t in range(T):
        dec0 = np.exp(G[:, :, t])  # decay of S0
        o_ref[:, :, t] = np.einsum("bhk,bhkv->bhv", qd[:, :, t] * dec0, S0)
        for s in range(t + 1):
            e = np.exp(G[:, :, t] - G[:, :, s])
            o_ref[:, :, t] += np.einsum("bhk,bhk->bh", qd[:, :, t] * e, kd[:, :, s])[..., None] * wv[:, :, s]
    assert maxabs(out, o_ref) < 1e-11


def test_recurrence_matches_transition_matrix_form():
    """Brute force with the paper's operator form (src/module.rs:76-78):
    S_t = (I - k_t (b_t*k_t)^T) diag(exp g_t) S_{t-1} + k_t (w_t*v_t)^T."""
    rng = np.random.default_rng(3)
    q, k, v, g, b, w = rand_inputs(rng, 1, 1, 1, 9, 5, 3, g_lo=-0.5, g_hi=0.0, b_hi=2.0)
    S0 = rng.standard_normal((1, 1, 5, 3))
    out, S = O.recurrent_f64(q, k, v, g, b, w, S0=S0, scale=0.5)
    St = S0[0, 0].copy()
    for t in range(9):
        kt = k[0, 0, t].astype(np.float64)
        M = np.eye(5) - np.outer(kt, b[0, 0, t] * kt)
        St = M @ np.diag(np.exp(g[0, 0, t].astype(np.float64))) @ St + np.outer(kt, w[0, 0, t].astype(np.float64) * v[0, 0, t])
        assert maxabs(out[0, 0, t], 0.5 * St.T @ q[0, 0, t]) < 1e-12
    assert maxabs(S[0, 0], St) < 1e-12


def test_recurrence_delta_rule_write_identity():
    """b = 1, g = 0, |k| = 1: one step makes k^T S equal w*v exactly."""
    rng = np.random.default_rng(4)
    q, k, v, g, b, w = rand_inputs(rng, 2, 2, 2, 1, 8, 6)
    g[:] = 0
    b[:] = 1
    S0 = rng.standard_normal((2, 2, 8, 6))
    _, S = O.recurrent_f64(q, k, v, g, b, w, S0=S0)
    kS = np.einsum("bhk,bhkv->bhv", k[:, :, 0].astype(np.float64), S)
    assert maxabs(kS, w[:, :, 0].astype(np.float64) * v[:, :, 0]) < 1e-6  # |k| = 1 to f32 rounding


def test_recurrence_negative_eigenvalue_reflection():
    """b = 2, g = 0, v = w = 0: S <- (I - 2 k k^T) S is a reflection, so two
    steps with the same key return S0 and the Frobenius norm is kept."""
    rng = np.random.default_rng(5)
    q, k, v, g, b, w = rand_inputs(rng, 1, 1, 1, 2, 8, 4)
    k[:, :, 1] = k[:, :, 0]
    kk = k.astype(np.float64)
    k = (kk / np.sqrt((kk * kk).sum(-1, keepdims=True))).astype(np.float32)
    g[:] = 0
    b[:] = 2
    v[:] = 0
    S0 = rng.standard_normal((1, 1, 8, 4))
    _, S1 = O.recurrent_f64(q[:, :, :1], k[:, :, :1], v[:, :, :1], g[:, :, :1], b[:, :, :1], w[:, :, :1], S0=S0)
    _, S2 = O.recurrent_f64(q, k, v, g, b, w, S0=S0)
    assert abs(np.linalg.norm(S1) - np.linalg.norm(S0)) < 1e-6
    assert maxabs(S2, S0) < 1e-6


def test_recurrence_f32_matches_f64():
    rng = np.random.default_rng(6)
    args = rand_inputs(rng, 2, 2, 4, 40, 16, 8)
    o64, S64 = O.recurrent_f64(*args, scale=0.25)
    o32, S32 = O.recurrent_f32(*args, scale=0.25)
    assert maxabs(o32, o64) < 1e-5 and maxabs(S32, S64) < 1e-5


def test_recurrence_head_repeat_equals_materialised():
    """Value head hv reads key head hv // rep; materialising the repeat gives the same result."""
    rng = np.random.default_rng(7)
    q, k, v, g, b, w = rand_inputs(rng, 2, 2, 6, 11, 8, 4)
    rep = 3
    mat = [np.repeat(a, rep, axis=1) for a in (q, k, g, b)]
    o1, S1 = O.recurrent_f64(q, k, v, g, b, w)
    o2, S2 = O.recurrent_f64(mat[0], mat[1], v, mat[2], mat[3], w)
    assert maxabs(o1, o2) == 0.0 and maxabs(S1, S2) == 0.0


# --------------------------------------------------------------------------
# chunked WY restatement (src/forward.rs:44-278)
# --------------------------------------------------------------------------
@pytest.mark.parametrize("decay", [(-0.3, -0.02), (-5.0, -0.5)])
@pytest.mark.parametrize("chunk", [16, 64])
def test_chunk_wy_stable_chunk_recipe(decay, chunk):
    """tests/stable_chunk.rs:11-63: scalar-per-head g, b broadcast, T = 96, tol 1e-3."""
    rng = np.random.default_rng(8)
    q, k, v, g, b, w = rand_inputs(rng, 2, 3, 3, 96, 8, 8, g_lo=decay[0], g_hi=decay[1], gdim=1, bdim=1)
    o_ref, S_ref = O.recurrent_f64(q, k, v, g, b, w, scale=1.0)
    o, S = O.chunk_wy_f32(q, k, v, g, b, w, scale=1.0, chunk_size=chunk)
    assert maxabs(o, o_ref) < 1e-3 and maxabs(S, S_ref) < 1e-3


def test_chunk_wy_real_decay_recipe():
    """tests/test_chunk.rs:200-256: per-channel g in U(-0.15,-0.01), random S0,
    T = 130 (ragged), K = 16, V = 8, C = 64, scale 0.125, tol 1e-4."""
    rng = np.random.default_rng(9)
    q, k, v, g, b, w = rand_inputs(rng, 2, 3, 3, 130, 16, 8, g_lo=-0.15, g_hi=-0.01)
    S0 = rng.standard_normal((2, 3, 16, 8)).astype(np.float32)
    o_ref, S_ref = O.recurrent_f64(q, k, v, g, b, w, S0=S0, scale=0.125)
    o, S = O.chunk_wy_f32(q, k, v, g, b, w, S0=S0, scale=0.125, chunk_size=64)
    assert maxabs(o, o_ref) < 1e-4 and maxabs(S, S_ref) < 1e-4


@pytest.mark.parametrize("chunk", [4, 8, 32, 128])
def test_chunk_wy_any_chunk_size_neg_eig(chunk):
    rng = np.random.default_rng(10)
    q, k, v, g, b, w = rand_inputs(rng, 1, 2, 4, 150, 16, 8, g_lo=-0.4, g_hi=-0.01, b_hi=2.0)
    o_ref, S_ref = O.recurrent_f64(q, k, v, g, b, w, scale=0.25)
    o, S = O.chunk_wy_f32(q, k, v, g, b, w, scale=0.25, chunk_size=chunk)
    assert maxabs(o, o_ref) < 1e-4 and maxabs(S, S_ref) < 1e-4


def test_chunk_wy_overflows_like_reference_at_strong_decay():
    """With |g| up to ~31 per token the k / exp(G - G_b) factor of the
    reference's tile-local scheme exceeds f32 range inside a 16-tile
    (src/forward.rs:170-184): the restatement yields non-finite values,
    as the reference does; the recurrence stays finite."""
    rng = np.random.default_rng(11)
    q, k, v, g, b, w = rand_inputs(rng, 1, 1, 1, 64, 16, 8, g_lo=-31.0, g_hi=-0.05)
    o_ref, _ = O.recurrent_f64(q, k, v, g, b, w)
    o, _ = O.chunk_wy_f32(q, k, v, g, b, w, chunk_size=64)
    assert np.all(np.isfinite(o_ref))
    assert not np.all(np.isfinite(o))


# --------------------------------------------------------------------------
# layer glue
# --------------------------------------------------------------------------
def test_short_conv_identity_and_shift_kernels():
    """Weights [0,0,0,1] give silu(x); weights [1,0,0,0] give silu(x[t-3])
    with the first row replicated before the sequence (src/short_conv.rs:42-54)."""
    rng = np.random.default_rng(12)
    x = rng.standard_normal((2, 7, 5))
    silu = lambda z: z / (1 + np.exp(-z))
    w_id = np.zeros((5, 4), np.float32)
    w_id[:, 3] = 1
    y, cache = O.short_conv(x, w_id)
    assert maxabs(y, silu(x)) < 1e-15
    assert maxabs(cache, x[:, -3:]) == 0
    w_sh = np.zeros((5, 4), np.float32)
    w_sh[:, 0] = 1
    y, _ = O.short_conv(x, w_sh)
    xp = np.concatenate([np.repeat(x[:, :1], 3, axis=1), x], axis=1)
    assert maxabs(y, silu(xp[:, :7])) < 1e-15


def test_short_conv_cache_continuation():
    rng = np.random.default_rng(13)
    x = rng.standard_normal((2, 11, 6))
    wc = rng.uniform(-0.5, 0.5, (6, 4)).astype(np.float32)
    y_full, c_full = O.short_conv(x, wc)
    y1, c1 = O.short_conv(x[:, :5], wc)
    y2, c2 = O.short_conv(x[:, 5:6], wc, c1)
    y3, c3 = O.short_conv(x[:, 6:], wc, c2)
    assert maxabs(np.concatenate([y1, y2, y3], axis=1), y_full) < 1e-14
    assert maxabs(c3, c_full) == 0
    # a sequence shorter than the cache: the cache still ends with the last 3 rows of pad|x
    _, c_short = O.short_conv(x[:, :2], wc)
    assert maxabs(c_short, np.concatenate([x[:, :1], x[:, :2]], axis=1)) == 0


def test_l2norm_and_rmsnorm_closed_forms():
    y = O.l2norm(np.array([[3.0, 4.0]]), eps=1e-6)
    assert maxabs(y, np.array([[3.0, 4.0]]) / np.sqrt(25.0 + 1e-6)) < 1e-15
    x = np.full((1, 8), 0.5)
    gate = np.zeros((1, 8))
    gate[0, 3] = 40.0  # silu(40) = 40 to double precision
    wn = np.arange(1, 9).astype(np.float32)
    y = O.rmsnorm_gate(x, gate, wn, eps=1e-5)
    expect = np.zeros((1, 8))
    expect[0, 3] = 0.5 / np.sqrt(0.25 + 1e-5) * 4.0 * 40.0
    assert maxabs(y, expect) < 1e-12


def _golden():
    z = np.load(GOLDEN)
    D, H, HK, HV, ev10, sc, ne = (int(t) for t in z["cfg"])
    cfg = Cfg(hidden_size=D, num_heads=H, head_dim=HK, expand_v=ev10 / 10, num_v_heads=HV,
              use_short_conv=bool(sc), allow_neg_eigval=bool(ne), norm_eps=float(z["norm_eps"][0]))
    W = {n: z[n] for n in O.WEIGHT_NAMES if n in z.files}
    return z, cfg, W


def test_layer_matches_reference_torch_model_golden_vectors():
    """Layer outputs vs the reference's pure-torch model (tests/gen_reference.py),
    42 cases, T in 1..38.  The reference's own tolerance is 5e-4
    (tests/bit_exact.rs); the double oracle lands at ~1e-7."""
    z, cfg, W = _golden()
    worst = 0.0
    for i in range(int(z["n_cases"][0])):
        r, _ = O.layer_forward(cfg, W, z[f"x{i}"])
        worst = max(worst, maxabs(r.out, z[f"y{i}"]))
    assert worst < 1e-5, worst


def test_layer_decode_equals_full_forward():
    """tests/autodiff.rs:31-66: token-by-token forward == one forward."""
    cfg = Cfg(hidden_size=32, num_heads=2, head_dim=16)
    W = init_weights(cfg, seed=3)
    x = np.random.default_rng(14).standard_normal((2, 12, 32)).astype(np.float32)
    full, _ = O.layer_forward(cfg, W, x)
    st = None
    outs = []
    for t in range(12):
        r, st = O.layer_forward(cfg, W, x[:, t:t + 1], state=st)
        outs.append(r.out)
    assert maxabs(np.concatenate(outs, axis=1), full.out) < 1e-12


def test_layer_prefill_then_decode():
    """tests/autodiff.rs:70-104 with a GVA, neg-eig, min_decay config."""
    cfg = Cfg(hidden_size=48, num_heads=2, head_dim=16, num_v_heads=4, expand_v=2.0, allow_neg_eigval=True,
              min_decay=0.9)
    W = init_weights(cfg, seed=4)
    x = np.random.default_rng(15).standard_normal((1, 9, 48)).astype(np.float32)
    full, st_full = O.layer_forward(cfg, W, x)
    _, st = O.layer_forward(cfg, W, x[:, :8])
    nxt, st = O.layer_forward(cfg, W, x[:, 8:], state=st)
    assert maxabs(nxt.out, full.out[:, 8:]) < 1e-12
    assert maxabs(st.recurrent, st_full.recurrent) < 1e-12


def test_layer_from_raw_is_the_layer_after_its_linears():
    cfg = Cfg(hidden_size=32, num_heads=2, head_dim=16, num_v_heads=4)
    W = init_weights(cfg, seed=5)
    x = np.random.default_rng(16).standard_normal((2, 5, 32)).astype(np.float32)
    full, st = O.layer_forward(cfg, W, x)
    xd = x.astype(np.float64)
    raw = {"q_raw": xd @ W["q_proj"], "k_raw": xd @ W["k_proj"], "v_raw": xd @ W["v_proj"],
           "f_raw": (xd @ W["f_proj_0"]) @ W["f_proj_1"], "b_raw": xd @ W["b_proj"], "w_raw": xd @ W["w_proj"],
           "gate": (xd @ W["g_proj_0"]) @ W["g_proj_1"] + W["g_proj_1_bias"]}
    on, oc, st2 = O.layer_from_raw(cfg, W, raw)
    assert maxabs(on @ W["o_proj"], full.out) < 1e-12
    assert maxabs(oc, full.o_core) < 1e-12 and maxabs(st2.recurrent, st.recurrent) < 1e-12


def test_layer_forward_f32_host_matches_layer_forward():
    """The f32 host layer (BLAS Linear layers + chunk_wy_f32; bench.py's CPU
    layer baseline) computes forward_train: ragged T, two batch rows."""
    cfg = Cfg(hidden_size=64, num_heads=2, head_dim=32, mode="chunk")
    W = init_weights(cfg, seed=6)
    x = np.random.default_rng(17).standard_normal((2, 100, 64)).astype(np.float32)
    full, _ = O.layer_forward(cfg, W, x)
    host = O.layer_forward_f32_host(cfg, W, x)
    assert host.dtype == np.float32 and host.shape == full.out.shape
    assert maxabs(host, full.out) <= 1e-4 * np.abs(full.out).max()
    with pytest.raises(ValueError):
        O.layer_forward_f32_host(Cfg(hidden_size=64, num_heads=2, head_dim=32, allow_neg_eigval=True), W, x)


def test_gva_reference_layout_scrambles_time():
    """The reference's unsqueeze/repeat/reshape (src/module.rs:459-463) maps
    value head h*rep+j at time t to key-side time (j*T + t) // rep: decode no
    longer reproduces prefill, while the head-repeat layout does; at T = 1 the
    two layouts coincide."""
    cfg = Cfg(hidden_size=32, num_heads=2, head_dim=8, num_v_heads=4)
    W = init_weights(cfg, seed=6)
    x = np.random.default_rng(17).standard_normal((1, 6, 32)).astype(np.float32)
    rep_full, _ = O.layer_forward(cfg, W, x, gva_scrambled=False)
    scr_full, _ = O.layer_forward(cfg, W, x, gva_scrambled=True)
    assert maxabs(rep_full.out, scr_full.out) > 1e-3
    one_r, _ = O.layer_forward(cfg, W, x[:, :1], gva_scrambled=False)
    one_s, _ = O.layer_forward(cfg, W, x[:, :1], gva_scrambled=True)
    assert maxabs(one_r.out, one_s.out) == 0.0

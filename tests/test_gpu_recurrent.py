"""GPU parity of the recurrent kernels against the double oracle.

Tolerance: max |error| <= 1e-4 on outputs and the final state (f32 bound of
the task, same as tests/test_chunk.rs:254-255)."""
import numpy as np
import pytest

from conftest import rand_inputs
from gdn2_testutil import Cfg, init_weights, maxabs
from oracle import oracle as O

TOL = 1e-4

pytestmark = pytest.mark.gpu


def _dev(gpu, *arrs):
    import torch

    return [torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(gpu) for a in arrs]


@pytest.mark.parametrize("B,Hk,HV,K,V", [(2, 4, 4, 128, 128), (3, 2, 4, 64, 64), (1, 2, 2, 128, 256),
                                         (2, 2, 2, 16, 24), (1, 1, 3, 32, 8), (2, 2, 2, 256, 64)])
def test_step_matches_recurrence(gpu, B, Hk, HV, K, V):
    """fused_step token by token == the per-token scan (tests/bench_cuda.rs:199-260 pattern)."""
    import gdn2_amd

    rng = np.random.default_rng(100 + K + V)
    T = 6
    q, k, v, g, b, w = rand_inputs(rng, B, Hk, HV, T, K, V, b_hi=2.0)
    S0 = rng.standard_normal((B, HV, K, V)).astype(np.float32) * 0.5
    o_ref, S_ref = O.recurrent_f64(q, k, v, g, b, w, S0=S0, scale=K ** -0.5)
    dq, dk, dv, dg, db, dw, dS = _dev(gpu, q, k, v, g, b, w, S0)
    state = dS
    for t in range(T):
        sl = lambda x: x[:, :, t:t + 1]
        res = gdn2_amd.fused_step(sl(dq), sl(dk), sl(dv), sl(dg), sl(db), sl(dw), state, K ** -0.5)
        assert res is not None
        o, state = res
        assert maxabs(o.cpu().numpy()[:, :, 0], o_ref[:, :, t]) < TOL
    assert maxabs(state.cpu().numpy(), S_ref) < TOL


def test_step_batch64_matches_oracle(gpu):
    """The bare step at the decode benchmark's shape (B = 64, 16 heads,
    K = V = 128, the streaming step kernel), three tokens in place on one
    state, against the double recurrence."""
    import gdn2_amd

    rng = np.random.default_rng(64)
    B, H, K, V, T = 64, 16, 128, 128, 3
    q, k, v, g, b, w = rand_inputs(rng, B, H, H, T, K, V, b_hi=1.0)
    q *= K ** -0.5 * 4
    S0 = rng.standard_normal((B, H, K, V)).astype(np.float32) * 0.3
    o_ref, S_ref = O.recurrent_f64(q, k, v, g, b, w, S0=S0, scale=K ** -0.5)
    dq, dk, dv, dg, db, dw, state = _dev(gpu, q, k, v, g, b, w, S0)
    for t in range(T):
        sl = lambda x: x[:, :, t:t + 1]
        o, state = gdn2_amd.fused_step(sl(dq), sl(dk), sl(dv), sl(dg), sl(db), sl(dw), state, K ** -0.5,
                                       out_state=state)
        e = maxabs(o.cpu().numpy()[:, :, 0], o_ref[:, :, t])
        assert e < TOL, (t, e)
    e_s = maxabs(state.cpu().numpy(), S_ref)
    print(f"B=64 step: final S err {e_s:.2e}")
    assert e_s < TOL


@pytest.mark.parametrize("B,Hk,HV,T,K,V", [(2, 4, 4, 64, 128, 128), (1, 2, 4, 37, 64, 128), (2, 2, 2, 20, 16, 24),
                                           (1, 1, 1, 300, 128, 128)])
def test_scan_matches_recurrence(gpu, B, Hk, HV, T, K, V):
    import gdn2_amd

    rng = np.random.default_rng(200 + T)
    q, k, v, g, b, w = rand_inputs(rng, B, Hk, HV, T, K, V)
    S0 = rng.standard_normal((B, HV, K, V)).astype(np.float32) * 0.5
    o_ref, S_ref = O.recurrent_f64(q, k, v, g, b, w, S0=S0, scale=0.3)
    dq, dk, dv, dg, db, dw, dS = _dev(gpu, q, k, v, g, b, w, S0)
    o, S = gdn2_amd.fused_recurrent_forward(dq, dk, dv, dg, db, dw, dS, 0.3)
    assert maxabs(o.cpu().numpy(), o_ref) < TOL
    assert maxabs(S.cpu().numpy(), S_ref) < TOL


def test_scan_in_place_and_strided_layout(gpu):
    """[B, T, H, D] views (strided heads) and an in-place state update."""
    import torch

    import gdn2_amd

    rng = np.random.default_rng(7)
    B, H, T, K, V = 2, 4, 33, 128, 128
    q, k, v, g, b, w = rand_inputs(rng, B, H, H, T, K, V)
    o_ref, S_ref = O.recurrent_f64(q, k, v, g, b, w, scale=0.1)
    bt = [torch.from_numpy(np.ascontiguousarray(a.transpose(0, 2, 1, 3))).to(gpu) for a in (q, k, v, g, b, w)]
    views = [x.permute(0, 2, 1, 3) for x in bt]  # [B, H, T, D] views of [B, T, H, D] storage
    S = torch.zeros((B, H, K, V), device=gpu)
    out = torch.empty((B, T, H, V), device=gpu).permute(0, 2, 1, 3)
    o, S2 = gdn2_amd.fused_recurrent_forward(*views, S, 0.1, out=out, in_place=True)
    assert S2.data_ptr() == S.data_ptr()
    assert maxabs(o.cpu().numpy(), o_ref) < TOL
    assert maxabs(S.cpu().numpy(), S_ref) < TOL


@pytest.mark.parametrize("T,update", [(1, True), (40, True), (40, False), (1, False)])
def test_fused_recurrent_gdn2_dispatch(gpu, T, update):
    """fused_recurrent_gdn2 (src/kernel/fused_recurrent.rs:65-108): state
    None = zeros, the fused step at T = 1, the scan otherwise; update_state
    False reads the state only (out = scale q S, permuted to [B, T, HV, V])
    and returns it unchanged."""
    import gdn2_amd

    B, Hk, HV, K, V = 2, 2, 4, 64, 128
    rng = np.random.default_rng(300 + T)
    q, k, v, g, b, w = rand_inputs(rng, B, Hk, HV, T, K, V)
    S0 = rng.standard_normal((B, HV, K, V)).astype(np.float32) * 0.5
    dq, dk, dv, dg, db, dw, dS = _dev(gpu, q, k, v, g, b, w, S0)
    o, S = gdn2_amd.fused_recurrent_gdn2(dq, dk, dv, dg, db, dw, dS, 0.3, update_state=update)
    if update:
        o_ref, S_ref = O.recurrent_f64(q, k, v, g, b, w, S0=S0, scale=0.3)
        assert maxabs(o.cpu().numpy(), o_ref) < TOL and maxabs(S.cpu().numpy(), S_ref) < TOL
        o0, S_zero = gdn2_amd.fused_recurrent_gdn2(dq, dk, dv, dg, db, dw, None, 0.3)  # None = zeros
        r0, Sr0 = O.recurrent_f64(q, k, v, g, b, w, S0=None, scale=0.3)
        assert maxabs(o0.cpu().numpy(), r0) < TOL and maxabs(S_zero.cpu().numpy(), Sr0) < TOL
    else:
        rep = HV // Hk
        qf = np.repeat(q.astype(np.float64), rep, axis=1)                 # [B, HV, T, K]
        ref = 0.3 * np.einsum("bhtk,bhkv->bhtv", qf, S0.astype(np.float64)).transpose(0, 2, 1, 3)
        assert tuple(o.shape) == (B, T, HV, V)
        assert maxabs(o.cpu().numpy(), ref) < TOL
        np.testing.assert_array_equal(S.cpu().numpy(), S0)


def _raw_from_layer(cfg, W, x):
    xd = x.astype(np.float64)
    return {"q_raw": xd @ W["q_proj"], "k_raw": xd @ W["k_proj"], "v_raw": xd @ W["v_proj"],
            "f_raw": (xd @ W["f_proj_0"]) @ W["f_proj_1"], "b_raw": xd @ W["b_proj"], "w_raw": xd @ W["w_proj"],
            "gate": (xd @ W["g_proj_0"]) @ W["g_proj_1"] + W["g_proj_1_bias"]}


@pytest.mark.parametrize("cfg", [
    Cfg(hidden_size=256, num_heads=2, head_dim=128),
    Cfg(hidden_size=256, num_heads=2, head_dim=128, num_v_heads=4, expand_v=2.0, allow_neg_eigval=True,
        min_decay=0.9),
    Cfg(hidden_size=64, num_heads=4, head_dim=16, expand_v=1.5),
    Cfg(hidden_size=128, num_heads=2, head_dim=64, use_short_conv=False),
], ids=["h128", "gva_v256_negeig_mindecay", "golden_shape_k16_v24", "k64_noconv"])
def test_decode_fused_matches_layer_from_raw(gpu, cfg):
    """Fused decode (conv, gates, L2 norm, step, gated RMSNorm) over 5 tokens
    == the double oracle of the layer after its Linear layers; first token
    without prior conv state (replicate padding), then with caches."""
    import torch

    import gdn2_amd

    B, T = 3, 5
    W = init_weights(cfg, seed=21)
    x = np.random.default_rng(22).standard_normal((B, T, cfg.hidden_size)).astype(np.float32)
    raw = _raw_from_layer(cfg, W, x)
    o_ref, _, st_ref = O.layer_from_raw(cfg, W, raw)
    params = {n: torch.from_numpy(W[n]).to(gpu) for n in ("q_conv_w", "k_conv_w", "v_conv_w", "a_log", "dt_bias",
                                                          "o_norm_weight")}
    if W["decay_factors"] is not None:
        params["decay_factors"] = torch.from_numpy(W["decay_factors"]).to(gpu)
    S = torch.zeros((B, cfg.hv, cfg.head_dim, cfg.v_head), device=gpu)
    caches = [tuple(torch.zeros((B, 3, n), device=gpu) for n in (cfg.kd, cfg.kd, cfg.vd)) for _ in range(2)]
    conv_in = None
    for t in range(T):
        rt = {n: torch.from_numpy(np.ascontiguousarray(a[:, t], np.float32)).to(gpu) for n, a in raw.items()}
        conv_out = caches[t % 2]
        out = gdn2_amd.decode_fused(rt, params, S, conv_in, conv_out, num_heads=cfg.num_heads, num_v_heads=cfg.hv,
                                    head_dim=cfg.head_dim, head_v_dim=cfg.v_head, scale=cfg.head_dim ** -0.5,
                                    min_decay=cfg.min_decay, norm_eps=cfg.norm_eps,
                                    use_short_conv=cfg.use_short_conv, allow_neg_eigval=cfg.allow_neg_eigval)
        conv_in = conv_out if cfg.use_short_conv else None
        assert maxabs(out.cpu().numpy(), o_ref[:, t]) < TOL, t
    assert maxabs(S.cpu().numpy(), st_ref.recurrent) < TOL
    if cfg.use_short_conv:
        for dev_c, ref_c in zip(conv_in, (st_ref.conv_q, st_ref.conv_k, st_ref.conv_v)):
            assert maxabs(dev_c.cpu().numpy(), ref_c) < 1e-5

"""GPU parity of the layer's backward (gdn2_layer_backward_f32) against the
oracle's double adjoint of GatedDeltaNet2 (oracle.layer_backward_f64, pinned
by finite differences in test_oracle_layer_bwd.py), on the layer's own
weights: the gradient of every parameter, of x and of the state on entry.
The reference gets these gradients from burn's autodiff
(tests/autodiff.rs:153-205); its tests check that they are nonzero, these
check their values.

Cases: short conv with ragged T, no short conv with a carried state and a
state gradient, GVA + negative eigenvalues + min_decay with a state, K = 128,
two tokens with a state (the conv cache straddles the call), gradient
accumulation, the torch autograd wrapper (loss = sum(out^2) / 2), and a
token-by-token decode chain run backwards through d_state == one backward
over the whole sequence.
Tolerance: max |error| <= REL * max |reference| + ABS for every tensor."""
import numpy as np
import pytest

from gdn2_testutil import maxabs
from oracle import oracle as O

REL = 1e-4
ABS = 1e-7

pytestmark = pytest.mark.gpu


def _close(got, ref, what, rel=REL):
    e = maxabs(got, ref)
    scale = float(np.abs(ref).max()) if np.size(ref) else 0.0
    print(f"  {what:16s} max|err|={e:.2e} max|ref|={scale:.3e}")
    assert e <= rel * scale + ABS, what


def _setup(gpu, over, seed=11):
    import gdn2_amd as G

    cfg = G.Gdn2Config(**over)
    layer = G.GatedDeltaNet2(cfg, seed=seed)
    rng = np.random.default_rng(seed + 100)
    # values away from the initialisers' constants, so that every term counts
    layer.set_param("o_norm_weight", rng.uniform(0.5, 1.5, cfg.v_head).astype(np.float32))
    layer.set_param("g_proj_1_bias", rng.normal(0, 1.0, cfg.vd).astype(np.float32))
    if cfg.min_decay is not None:
        layer.set_param("decay_factors", rng.normal(0, 1.0, cfg.num_heads * cfg.head_dim).astype(np.float32))
    return G, cfg, layer, layer.params()


def _rand_state(G, layer, rng, B, cfg):
    st = G.Gdn2State(layer, B)
    arrs = [rng.normal(0, 0.3, (B, cfg.hv, cfg.head_dim, cfg.v_head)), rng.normal(0, 1.0, (B, 3, cfg.kd)),
            rng.normal(0, 1.0, (B, 3, cfg.kd)), rng.normal(0, 1.0, (B, 3, cfg.vd))]
    arrs = [a.astype(np.float32) for a in arrs]
    for i, a in enumerate(arrs):
        st.write(i, a)
    return st, O.OracleState(*(a.astype(np.float64) for a in arrs))


def _compare(grads, dx, d_state_in, ref, names, rel=None):
    """rel: per-parameter relative bounds that replace REL."""
    for n in names:
        g, r = grads.get(n), ref.params[n]
        if r is None:
            assert g is None, n
            continue
        _close(g, r, n, (rel or {}).get(n, REL))
    if dx is not None:
        _close(dx.cpu().numpy(), ref.dx, "dx")
    if d_state_in is not None:
        for i, f in enumerate(("recurrent", "conv_q", "conv_k", "conv_v")):
            _close(d_state_in.read(i), getattr(ref.d_state, f), "d_state." + f)


SMALL = dict(hidden_size=256, num_heads=4, head_dim=64, mode="chunk")
CASES = {
    # id: config, B, T, carried state, state gradient
    "conv_ragged": (SMALL, 2, 150, False, False),
    "no_conv_state": (dict(SMALL, use_short_conv=False), 2, 70, True, True),
    "gva_negeig_mindecay_state": (dict(hidden_size=256, num_heads=2, num_v_heads=4, head_dim=64, expand_v=2.0,
                                       allow_neg_eigval=True, min_decay=0.9, mode="chunk"), 2, 100, True, True),
    "k128": (dict(hidden_size=512, num_heads=2, head_dim=128, mode="fused_recurrent"), 1, 300, False, False),
    "T2_state": (SMALL, 2, 2, True, True),
    # the reference's CPU-benchmark layer (tests/bit_exact.rs:224-235): V = 96
    "v96": (dict(SMALL, expand_v=1.5), 2, 130, False, True),
    "k32": (dict(hidden_size=128, num_heads=4, head_dim=32, mode="chunk"), 1, 200, True, False),
}


@pytest.mark.parametrize("name", list(CASES))
def test_layer_backward_matches_oracle(gpu, name):
    import torch

    over, B, T, carried, with_ds = CASES[name]
    G, cfg, layer, W = _setup(gpu, over)
    rng = np.random.default_rng(5)
    xh = rng.standard_normal((B, T, cfg.hidden_size)).astype(np.float32)
    dh = rng.standard_normal((B, T, cfg.hidden_size)).astype(np.float32)
    st, ost = _rand_state(G, layer, rng, B, cfg) if carried else (None, None)
    ds, ods = _rand_state(G, layer, rng, B, cfg) if with_ds else (None, None)
    print(f"case {name}: B={B} T={T}", flush=True)
    dx, grads, dsi = layer.backward(torch.from_numpy(xh).to(gpu), torch.from_numpy(dh).to(gpu), state=st,
                                    d_state=ds, want_d_state=True)
    ref = O.layer_backward_f64(cfg, W, xh, dh, ost, ods)
    _compare(grads, dx, dsi, ref, O.WEIGHT_NAMES)
    if st is not None:  # state_in is read only
        np.testing.assert_array_equal(st.read(0), ost.recurrent.astype(np.float32))


def test_accumulate_adds(gpu):
    import torch

    G, cfg, layer, W = _setup(gpu, SMALL)
    rng = np.random.default_rng(8)
    B, T = 1, 90
    x1, x2 = (rng.standard_normal((B, T, cfg.hidden_size)).astype(np.float32) for _ in range(2))
    d1, d2 = (rng.standard_normal((B, T, cfg.hidden_size)).astype(np.float32) for _ in range(2))
    t = lambda a: torch.from_numpy(a).to(gpu)
    _, grads, _ = layer.backward(t(x1), t(d1), want_dx=False)
    layer.backward(t(x2), t(d2), grads=grads, accumulate=True, want_dx=False)
    r1 = O.layer_backward_f64(cfg, W, x1, d1)
    r2 = O.layer_backward_f64(cfg, W, x2, d2)
    for n in O.WEIGHT_NAMES:
        if r1.params[n] is not None:
            _close(grads.get(n), r1.params[n] + r2.params[n], n)
    grads.zero()
    assert all(np.all(g == 0) for g in grads.as_dict().values() if g is not None)


def test_autograd_wrapper(gpu):
    """loss = sum(out^2) / 2 through torch autograd: x.grad and layer.grads
    equal the adjoint with d_out = out (tests/autodiff.rs:153-175 pattern)."""
    import torch

    G, cfg, layer, W = _setup(gpu, dict(SMALL, mode="fused_recurrent"))
    rng = np.random.default_rng(9)
    xh = rng.standard_normal((2, 24, cfg.hidden_size)).astype(np.float32)
    x = torch.from_numpy(xh).to(gpu).requires_grad_(True)
    out = layer.forward_train_autograd(x)
    loss = 0.5 * (out * out).sum()
    loss.backward()
    ref = O.layer_backward_f64(cfg, W, xh, out.detach().cpu().numpy().astype(np.float64))
    assert float(np.abs(layer.grads.get("q_proj")).max()) > 0 and float(np.abs(layer.grads.get("a_log")).max()) > 0
    _compare(layer.grads, x.grad, None, ref, O.WEIGHT_NAMES)


def test_decode_chain_backward_equals_one_pass(gpu):
    """Token-by-token forward calls with a state (tests/autodiff.rs:177-205),
    differentiated backwards call by call with d_state = the next call's
    d_state_in and accumulate = 1, equal one backward over the sequence."""
    import torch

    G, cfg, layer, W = _setup(gpu, dict(SMALL, mode="fused_recurrent"))
    rng = np.random.default_rng(10)
    B, T = 2, 6
    x = torch.from_numpy(rng.standard_normal((B, T, cfg.hidden_size)).astype(np.float32)).to(gpu)
    d = torch.from_numpy(rng.standard_normal((B, T, cfg.hidden_size)).astype(np.float32)).to(gpu)
    state, before = G.Gdn2State(layer, B), []
    for t in range(T):
        before.append(G.Gdn2State.from_bytes(layer, state.to_bytes()) if state.is_some else None)
        layer.forward(x[:, t:t + 1].contiguous(), state)
    grads, d_state, dxs = G.Gdn2Grads(layer), None, [None] * T
    for t in reversed(range(T)):
        dxs[t], _, d_state = layer.backward(x[:, t:t + 1].contiguous(), d[:, t:t + 1].contiguous(), state=before[t],
                                            d_state=d_state, grads=grads, accumulate=True, want_d_state=True)
    dx_one, g_one, dsi_one = layer.backward(x, d, want_d_state=True)
    for n in O.WEIGHT_NAMES:
        a, b = grads.get(n), g_one.get(n)
        if b is not None:
            _close(a, b, n)
    _close(torch.cat(dxs, dim=1).cpu().numpy(), dx_one.cpu().numpy(), "dx")
    _close(d_state.read(0), dsi_one.read(0), "dS0")


@pytest.mark.parametrize("mode", ["fused_recurrent", "chunk"])
def test_small_heads_backward_matches_oracle(gpu, mode):
    """The reference's gradient test configuration (tests/autodiff.rs:153-175:
    hidden 32, 2 heads of 16, B = 2, T = 24, both modes): heads the chunked
    backward does not take run the scan's adjoint."""
    import torch

    G, cfg, layer, W = _setup(gpu, dict(hidden_size=32, num_heads=2, head_dim=16, mode=mode))
    rng = np.random.default_rng(21)
    B, T = 2, 24
    xh = rng.standard_normal((B, T, cfg.hidden_size)).astype(np.float32)
    dh = rng.standard_normal((B, T, cfg.hidden_size)).astype(np.float32)
    dx, grads, dsi = layer.backward(torch.from_numpy(xh).to(gpu), torch.from_numpy(dh).to(gpu), want_d_state=True)
    ref = O.layer_backward_f64(cfg, W, xh, dh)
    assert float(np.abs(grads.get("q_proj")).max()) > 0 and float(np.abs(grads.get("a_log")).max()) > 0
    _compare(grads, dx, dsi, ref, O.WEIGHT_NAMES)


def test_head_dim_256_backward_matches_oracle(gpu):
    """head_dim 256 (K = V = 256, two heads): the chunked backward's K = 256
    kernels, every gradient against the double adjoint."""
    import torch

    G, cfg, layer, W = _setup(gpu, dict(hidden_size=512, num_heads=2, head_dim=256, mode="chunk"))
    rng = np.random.default_rng(17)
    B, T = 1, 150
    xh = rng.standard_normal((B, T, cfg.hidden_size)).astype(np.float32)
    dh = rng.standard_normal((B, T, cfg.hidden_size)).astype(np.float32)
    dx, grads, dsi = layer.backward(torch.from_numpy(xh).to(gpu), torch.from_numpy(dh).to(gpu), want_d_state=True)
    ref = O.layer_backward_f64(cfg, W, xh, dh)
    _compare(grads, dx, dsi, ref, O.WEIGHT_NAMES)


def test_backward_rejects_oversized_heads(gpu):
    import torch

    G = pytest.importorskip("gdn2_amd")
    cfg = G.Gdn2Config(hidden_size=512, num_heads=1, head_dim=512)  # K = V = 512: neither backward kernel
    layer = G.GatedDeltaNet2(cfg)
    x = torch.zeros((1, 4, 512), device=gpu)
    with pytest.raises(G._capi.Gdn2Error) as e:
        layer.backward(x, x)
    assert e.value.status == G._capi.GDN2_NOT_APPLICABLE


@pytest.mark.parametrize("strong", [False, True], ids=["min_decay", "dt_bias_plus_4"])
def test_saved_activations_equal_recompute(gpu, strong):
    """forward_train with saved activations (which also keeps the chunked
    recurrence's per-chunk quantities: gdn2_chunk_fwd_train_f32) gives the
    same output as without, and the backward from them
    (gdn2_chunk_bwd_saved_f32) equals the recomputing backward bit for bit;
    also with decays strong enough that diagonal-block channels take the
    exact pairwise path."""
    import torch

    over = dict(SMALL, hidden_size=256, num_heads=2, head_dim=128) if strong else \
        dict(SMALL, min_decay=0.9, allow_neg_eigval=True)
    G, cfg, layer, W = _setup(gpu, over)
    if strong:
        layer.set_param("dt_bias", W["dt_bias"] + 4.0)
    rng = np.random.default_rng(12)
    B, T = 2, 130
    x = torch.from_numpy(rng.standard_normal((B, T, cfg.hidden_size)).astype(np.float32)).to(gpu)
    d = torch.from_numpy(rng.standard_normal((B, T, cfg.hidden_size)).astype(np.float32)).to(gpu)
    if strong:  # the case reaches the masked channels
        gt = layer.project(x)["g"].cpu().numpy().astype(np.float64)
        gt = np.pad(gt, [(0, 0), (0, 0), (0, (-T) % 16), (0, 0)])
        assert (-gt.reshape(B, cfg.num_heads, -1, 16, cfg.head_dim).sum(3) * np.log2(np.e) > 96).any()
    saved = G.Gdn2Saved(layer, B, T)
    out_s = layer.forward_train(x, saved=saved)
    out_r = layer.forward_train(x)
    assert torch.equal(out_s, out_r)
    dx_s, g_s, _ = layer.backward(x, d, saved=saved)
    dx_r, g_r, _ = layer.backward(x, d)
    assert torch.equal(dx_s, dx_r)
    for n in O.WEIGHT_NAMES:
        a, b = g_s.get(n), g_r.get(n)
        if b is not None:
            np.testing.assert_array_equal(a, b, err_msg=n)
    with pytest.raises(G._capi.Gdn2Error):  # shape mismatch
        layer.backward(x[:, :64].contiguous(), d[:, :64].contiguous(), saved=saved)


def test_strong_decay_layer_backward(gpu):
    """The long-context configuration's decays (dt_bias + 4: per-token |g| of
    tens) on a small layer in chunk mode: the training forward's and the
    backward's diagonal blocks with 16-token decay spans in (96, 192] (the
    mid-tile reference) and above 192 (half-block products and exact pairwise
    terms) are reached (asserted on the layer's own g) and every gradient
    matches the double adjoint."""
    import torch

    G, cfg, layer, W = _setup(gpu, dict(SMALL, hidden_size=256, num_heads=2, head_dim=128))
    layer.set_param("dt_bias", W["dt_bias"] + 4.0)
    W = layer.params()
    rng = np.random.default_rng(15)
    B, T = 2, 100
    xh = rng.standard_normal((B, T, cfg.hidden_size)).astype(np.float32)
    dh = rng.standard_normal((B, T, cfg.hidden_size)).astype(np.float32)
    x = torch.from_numpy(xh).to(gpu)
    g = layer.project(x)["g"].cpu().numpy()
    gt = np.pad(g.astype(np.float64), [(0, 0), (0, 0), (0, (-T) % 16), (0, 0)])
    half = -gt.reshape(B, cfg.num_heads, -1, 2, 8, cfg.head_dim).sum(4) * np.log2(np.e)
    span, hmax = half.sum(3), half.max(3)
    mid = int(((span > 96) & (span <= 192)).sum())
    split, pair = int(((span > 192) & (hmax <= 192)).sum()), int(((span > 192) & (hmax > 192)).sum())
    print(f"tiles x channels with spans in (96, 192]: {mid}, above 192 in halves of at most 192: {split}, "
          f"other: {pair}, of {span.size}")
    assert mid > 0 and split > 0 and pair > 0
    dx, grads, dsi = layer.backward(x, torch.from_numpy(dh).to(gpu), want_d_state=True)
    ref = O.layer_backward_f64(cfg, W, xh, dh)
    # A_log's gradient is sum(dg g) with per-token |g| up to ~28 here: the f32
    # rounding of dg (seen at ~2e-5 relative in dt_bias's gradient, sum(dg dg/d dt_bias)
    # with |dg/d dt_bias| <= e^A_log) comes back scaled by |g|, ~1e-4 relative
    _compare(grads, dx, dsi, ref, O.WEIGHT_NAMES, rel={"a_log": 2.5e-4})

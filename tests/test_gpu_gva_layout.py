"""GPU parity of the layer in the reference's GVA layout (gva_layout =
"reference": src/module.rs:456-468, value head h rep + a at time t reads key
head h at time (a T + t) / rep of the same call) against the oracle run with
gva_scrambled: forward_train in both modes, forward calls carrying a state
(each call scrambled within itself, as the reference does per call),
project()'s [B, HV, T, K] outputs, and the backward (chunked and per-token,
recomputed and from saved activations) against the double adjoint.
Tolerances: those of test_gpu_layer.py (forward) and test_gpu_layer_bwd.py
(backward)."""
import numpy as np
import pytest

from gdn2_testutil import maxabs
from oracle import oracle as O

TOL = 1e-4
REL = 1e-4
ABS = 1e-7

pytestmark = pytest.mark.gpu

GVA = dict(hidden_size=256, num_heads=2, num_v_heads=4, head_dim=64, expand_v=2.0, allow_neg_eigval=True,
           min_decay=0.9, gva_layout="reference")


def _layer(over, seed=11):
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


def _x(gpu, seed, B, T, D):
    import torch

    xh = np.random.default_rng(seed).standard_normal((B, T, D)).astype(np.float32)
    return xh, torch.from_numpy(xh).to(gpu)


def _close(got, ref, what):
    e = maxabs(got, ref)
    scale = float(np.abs(ref).max())
    print(f"{what} max|err|={e:.2e} max|ref|={scale:.3e}")
    assert e < TOL and e <= REL * scale, what


@pytest.mark.parametrize("mode,B,T", [("chunk", 2, 150), ("fused_recurrent", 2, 40), ("chunk", 1, 300)],
                         ids=["chunk", "recurrent", "chunk_T300"])
def test_forward_train_reference_layout(gpu, mode, B, T):
    """forward_train against the oracle in the reference's layout; the
    head-repeat oracle differs (the layouts are not the same map)."""
    G, cfg, layer, W = _layer(dict(GVA, mode=mode))
    xh, x = _x(gpu, 3, B, T, cfg.hidden_size)
    out = layer.forward_train(x).cpu().numpy()
    ref, _ = O.layer_forward(cfg, W, xh, gva_scrambled=True)
    _close(out, ref.out, "out")
    rep, _ = O.layer_forward(cfg, W, xh, gva_scrambled=False)
    assert maxabs(ref.out, rep.out) > 10 * TOL * max(1.0, float(np.abs(ref.out).max()))


def test_project_reference_layout(gpu):
    """project()'s q, k, g, b are [B, HV, T, K] in the reference's layout:
    bit-identical to the head-repeat layer's [B, H, T, K] outputs put through
    the reference's unsqueeze/repeat/reshape, and within the tolerance of the
    oracle's."""
    import gdn2_amd as G

    _, cfg, layer, W = _layer(GVA, seed=5)
    head = G.GatedDeltaNet2(G.Gdn2Config(**dict(GVA, gva_layout="head_repeat")), seed=5)
    head.load_params(W)
    B, T = 2, 37
    xh, x = _x(gpu, 4, B, T, cfg.hidden_size)
    p = {n: t.cpu().numpy() for n, t in layer.project(x).items()}
    h = {n: t.cpu().numpy() for n, t in head.project(x).items()}
    ref, _ = O.layer_forward(cfg, W, xh, gva_scrambled=True, want_proj=True)
    rep = cfg.hv // cfg.num_heads
    for n in ("q", "k", "g", "b"):
        assert p[n].shape == (B, cfg.hv, T, cfg.head_dim), n
        expanded = np.repeat(h[n][:, :, :, None, :], rep, axis=3).reshape(p[n].shape)
        assert np.array_equal(p[n], expanded), n
        assert maxabs(p[n], ref.proj[n]) < TOL, n
    for n in ("v", "w", "gate"):
        assert np.array_equal(p[n], h[n]), n


def test_forward_calls_with_state_reference_layout(gpu):
    """A 130-token call, then single tokens, then a 20-token call, carrying
    the state: each call in the reference's layout within itself (the
    single tokens coincide with head repeat), against the oracle call by
    call from the same states."""
    import torch

    _, cfg, layer, W = _layer(dict(GVA, mode="chunk"), seed=21)
    B = 2
    xh, x = _x(gpu, 9, B, 130 + 3 + 20, cfg.hidden_size)
    st, ost = None, None
    for a, b in ((0, 130), (130, 131), (131, 132), (132, 133), (133, 153)):
        out, st = layer.forward(x[:, a:b].contiguous(), st)
        ref, ost = O.layer_forward(cfg, W, xh[:, a:b], state=ost, gva_scrambled=True)
        _close(out.cpu().numpy(), ref.out, f"tokens [{a}, {b})")
    torch.cuda.synchronize()
    assert maxabs(st.recurrent, ost.recurrent) < TOL
    for n in ("conv_q", "conv_k", "conv_v"):
        assert maxabs(getattr(st, n), getattr(ost, n)) < TOL, n


def _bwd_close(got, ref, what):
    e = maxabs(got, ref)
    scale = float(np.abs(ref).max()) if np.size(ref) else 0.0
    print(f"  {what:16s} max|err|={e:.2e} max|ref|={scale:.3e}")
    assert e <= REL * scale + ABS, what


@pytest.mark.parametrize("mode,B,T,saved", [("chunk", 2, 100, False), ("chunk", 2, 100, True),
                                            ("fused_recurrent", 1, 30, False)],
                         ids=["chunk", "chunk_saved", "recurrent"])
def test_backward_reference_layout(gpu, mode, B, T, saved):
    """Every parameter's gradient and dx against the oracle's double adjoint
    in the reference's layout (each key element's rep copies summed)."""
    import torch

    G, cfg, layer, W = _layer(dict(GVA, mode=mode))
    xh, x = _x(gpu, 15, B, T, cfg.hidden_size)
    dh = np.random.default_rng(16).standard_normal((B, T, cfg.hidden_size)).astype(np.float32)
    acts = None
    if saved:
        acts = G.Gdn2Saved(layer, B, T)
        layer.forward_train(x, saved=acts)
    dx, grads, _ = layer.backward(x, torch.from_numpy(dh).to(gpu), saved=acts)
    ref = O.layer_backward_f64(cfg, W, xh, dh, gva_scrambled=True)
    for n in O.WEIGHT_NAMES:
        r = ref.params[n]
        if r is None:
            assert grads.get(n) is None, n
            continue
        _bwd_close(grads.get(n), r, n)
    _bwd_close(dx.cpu().numpy(), ref.dx, "dx")

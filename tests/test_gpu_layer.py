"""GPU parity of the whole layer (include/gdn2_layer.h) against the oracle's
double restatement of GatedDeltaNet2 (src/module.rs:224-495), fed the
layer's own seeded weights.

Checks: forward_train in both modes, project() outputs, forward() with a
state (prefill then token-by-token decode == one pass over the whole
sequence, src/module.rs:224-316 + tests/autodiff.rs:31-104), Option::None
vs Gdn2State::zeros, no short conv, GVA + negative eigenvalues + min_decay.
Tolerance: max |error| <= 1e-4 on outputs and on the final state
(tests/test_chunk.rs:254-255).  The layer output at these initialisations
is small (|out| ~ 1e-2: silu of a near-zero gate times Xavier-scaled
o_proj), so the outputs are also held to a relative bound,
max |error| <= REL * max |reference|."""
import numpy as np
import pytest

from gdn2_testutil import maxabs
from oracle import oracle as O

TOL = 1e-4
REL = 1e-4

pytestmark = pytest.mark.gpu


def _close(got, ref, what=""):
    e = maxabs(got, ref)
    scale = float(np.abs(ref).max())
    print(f"{what} max|err|={e:.2e} max|ref|={scale:.3e} rel={e / max(scale, 1e-30):.2e}")
    assert e < TOL and e <= REL * scale, what


def _oracle_state(st):
    return O.OracleState(st.recurrent, st.conv_q, st.conv_k, st.conv_v)


def _x(gpu, rng, B, T, D):
    import torch

    xh = rng.standard_normal((B, T, D)).astype(np.float32)
    return xh, torch.from_numpy(xh).to(gpu)


SMALL = dict(hidden_size=256, num_heads=4, head_dim=64)

CASES = {
    # config 1 of the benchmark list: D 256, 4 heads, K = V = 64, chunk, short conv
    "c1_chunk": (dict(SMALL, mode="chunk"), 1, 1024),
    "c1_recurrent": (dict(SMALL, mode="fused_recurrent"), 2, 150),
    "no_conv_chunk": (dict(SMALL, mode="chunk", use_short_conv=False), 2, 130),
    "gva_negeig_mindecay": (dict(hidden_size=256, num_heads=2, num_v_heads=4, head_dim=64, expand_v=2.0,
                                 allow_neg_eigval=True, min_decay=0.9, mode="chunk"), 2, 200),
    "k128_chunk": (dict(hidden_size=512, num_heads=2, head_dim=128, mode="chunk"), 1, 300),
    "k256_chunk": (dict(hidden_size=512, num_heads=2, head_dim=256, mode="chunk"), 2, 200),
    "k256_v128_gva": (dict(hidden_size=512, num_heads=1, num_v_heads=2, head_dim=256, expand_v=0.5, mode="chunk"),
                      1, 150),
    # at most 256 rows: the rank-256 up-projections take the one-launch MFMA kernel
    "k256_few_rows": (dict(hidden_size=512, num_heads=2, head_dim=256, mode="chunk"), 2, 100),
    # the reference's CPU benchmark model (tests/bit_exact.rs:224-235: D 256, 4 heads, K 64,
    # expand_v 1.5, both modes): V = 96 on the chunk kernels' three 32-column slices
    "bench_v96_chunk": (dict(hidden_size=256, num_heads=4, head_dim=64, expand_v=1.5, mode="chunk"), 2, 300),
    "bench_v96_recurrent": (dict(hidden_size=256, num_heads=4, head_dim=64, expand_v=1.5,
                                 mode="fused_recurrent"), 1, 256),
    # the reference's "tiny" and "small" CUDA benchmark layers (tests/bench_cuda.rs:71-72: K = V = 32)
    "bench_tiny": (dict(hidden_size=64, num_heads=2, head_dim=32, mode="chunk"), 1, 200),
    "bench_small": (dict(hidden_size=128, num_heads=4, head_dim=32, mode="chunk"), 2, 256),
    "k128_v192": (dict(hidden_size=512, num_heads=2, head_dim=128, expand_v=1.5, mode="chunk"), 1, 200),
}


@pytest.mark.parametrize("name", list(CASES))
def test_forward_train_matches_oracle(gpu, name):
    import gdn2_amd as G

    over, B, T = CASES[name]
    cfg = G.Gdn2Config(**over)
    layer = G.GatedDeltaNet2(cfg, seed=11)
    W = layer.params()
    xh, x = _x(gpu, np.random.default_rng(3), B, T, cfg.hidden_size)
    out = layer.forward_train(x).cpu().numpy()
    ref, _ = O.layer_forward(cfg, W, xh)
    _close(out, ref.out, name)


def test_project_matches_oracle(gpu):
    import gdn2_amd as G

    cfg = G.Gdn2Config(hidden_size=256, num_heads=2, num_v_heads=4, head_dim=64, expand_v=2.0, allow_neg_eigval=True,
                       min_decay=0.9, mode="chunk")
    layer = G.GatedDeltaNet2(cfg, seed=5)
    W = layer.params()
    B, T = 2, 37
    xh, x = _x(gpu, np.random.default_rng(4), B, T, cfg.hidden_size)
    p = {n: t.cpu().numpy() for n, t in layer.project(x).items()}
    ref, _ = O.layer_forward(cfg, W, xh, want_proj=True)
    for n in ("q", "k", "g", "b", "v", "w"):
        e = maxabs(p[n], ref.proj[n])  # both [B, H, T, D]
        print(f"{n}: {e:.2e}")
        assert e < TOL, n
    assert maxabs(p["gate"], ref.proj["gate"]) < TOL


@pytest.mark.parametrize("over", [dict(SMALL, mode="chunk"),
                                  dict(hidden_size=256, num_heads=2, num_v_heads=4, head_dim=64, expand_v=2.0,
                                       allow_neg_eigval=True, min_decay=0.9, mode="chunk"),
                                  dict(SMALL, mode="fused_recurrent", use_short_conv=False)],
                         ids=["c1", "gva_negeig_mindecay", "recurrent_noconv"])
def test_prefill_then_decode_equals_one_pass(gpu, over):
    """forward(prefill) then T single-token forward calls == the oracle's one
    pass over the whole sequence, on every output and on S and the conv
    caches at the end."""
    import torch

    import gdn2_amd as G

    cfg = G.Gdn2Config(**over)
    layer = G.GatedDeltaNet2(cfg, seed=21)
    W = layer.params()
    B, Tp, Td = 2, 130, 12
    xh, x = _x(gpu, np.random.default_rng(9), B, Tp + Td, cfg.hidden_size)
    ref, rst = O.layer_forward(cfg, W, xh)
    out_p, st = layer.forward(x[:, :Tp])
    outs = [out_p]
    for t in range(Tp, Tp + Td):
        o, st = layer.forward(x[:, t:t + 1].contiguous(), st)
        outs.append(o)
    out = torch.cat(outs, 1).cpu().numpy()
    _close(out, ref.out, "out")
    es = maxabs(st.recurrent, rst.recurrent)
    print(f"S {es:.2e}")
    assert es < TOL
    if cfg.use_short_conv:
        for n in ("conv_q", "conv_k", "conv_v"):
            assert maxabs(getattr(st, n), getattr(rst, n)) < TOL, n
    else:
        assert not np.any(st.conv_q) and not np.any(st.conv_v)


def test_short_inputs_take_the_recurrent_rule_and_continue(gpu):
    """Three calls of 40, 1 and 64 tokens (<= 64: the recurrent path) carry
    S and the conv caches like one call over 105 tokens."""
    import torch

    import gdn2_amd as G

    cfg = G.Gdn2Config(**dict(SMALL, mode="chunk"))
    layer = G.GatedDeltaNet2(cfg, seed=2)
    W = layer.params()
    xh, x = _x(gpu, np.random.default_rng(12), 1, 105, cfg.hidden_size)
    ref, rst = O.layer_forward(cfg, W, xh)
    o1, st = layer.forward(x[:, :40].contiguous())
    o2, st = layer.forward(x[:, 40:41].contiguous(), st)
    o3, st = layer.forward(x[:, 41:].contiguous(), st)
    out = torch.cat([o1, o2, o3], 1).cpu().numpy()
    _close(out, ref.out, "out")
    assert maxabs(st.recurrent, rst.recurrent) < TOL
    assert maxabs(st.conv_v, rst.conv_v) < TOL


def test_zeros_state_differs_from_none_like_reference(gpu):
    """Gdn2State::zeros pads the conv with zeros, Option::None with the first
    token (src/short_conv.rs:30-56); both match the oracle."""
    import gdn2_amd as G

    cfg = G.Gdn2Config(**dict(SMALL, mode="chunk"))
    layer = G.GatedDeltaNet2(cfg, seed=4)
    W = layer.params()
    xh, x = _x(gpu, np.random.default_rng(13), 2, 80, cfg.hidden_size)
    o_none, _ = layer.forward(x)
    z = G.Gdn2State.zeros(layer, 2)
    o_zero, z = layer.forward(x, z)
    ref_none, _ = O.layer_forward(cfg, W, xh)
    zero_state = O.OracleState(*(np.zeros(s) for s in ((2, cfg.hv, 64, 64), (2, 3, 256), (2, 3, 256), (2, 3, 256))))
    ref_zero, _ = O.layer_forward(cfg, W, xh, state=zero_state)
    _close(o_none.cpu().numpy(), ref_none.out, "none")
    _close(o_zero.cpu().numpy(), ref_zero.out, "zeros")
    assert maxabs(ref_none.out, ref_zero.out) > 0.05 * np.abs(ref_none.out).max()


def test_state_written_from_host_is_used(gpu):
    """A state restored through gdn2_state_write continues like the oracle
    started from the same S and caches."""
    import gdn2_amd as G

    cfg = G.Gdn2Config(**dict(SMALL, mode="chunk"))
    layer = G.GatedDeltaNet2(cfg, seed=8)
    W = layer.params()
    rng = np.random.default_rng(14)
    B = 2
    st = G.Gdn2State(layer, B)
    assert not st.is_some
    S0 = (rng.standard_normal((B, 4, 64, 64)) * 0.3).astype(np.float32)
    cq, ck, cv = (rng.standard_normal((B, 3, 256)).astype(np.float32) for _ in range(3))
    for which, a in ((st.RECURRENT, S0), (st.CONV_Q, cq), (st.CONV_K, ck), (st.CONV_V, cv)):
        st.write(which, a)
    assert st.is_some
    xh, x = _x(gpu, rng, B, 70, cfg.hidden_size)
    out, st = layer.forward(x, st)
    ref, rst = O.layer_forward(cfg, W, xh, state=O.OracleState(S0, cq, ck, cv))
    _close(out.cpu().numpy(), ref.out, "out")
    assert maxabs(st.recurrent, rst.recurrent) < TOL


def test_layer_errors(gpu):
    import torch

    import gdn2_amd as G
    from gdn2_amd._capi import Gdn2Error

    cfg = G.Gdn2Config(**SMALL)
    layer = G.GatedDeltaNet2(cfg, seed=1)
    with pytest.raises(ValueError, match="expected hidden_states with last dim 256 but got 128"):
        layer.forward_train(torch.zeros((1, 4, 128), device=gpu))
    st = G.Gdn2State(layer, 2)
    with pytest.raises(Gdn2Error, match="state batch 2 != input batch 1"):
        layer.forward(torch.zeros((1, 4, 256), device=gpu), st)
    with pytest.raises(ValueError):
        G.GatedDeltaNet2(G.Gdn2Config(num_heads=3, num_v_heads=4))

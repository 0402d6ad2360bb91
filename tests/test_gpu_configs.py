"""The benchmark configurations at their full sizes, on the GPU.

At these sizes the oracle cannot run the whole batch in seconds, so each
configuration is held to size-independent properties plus oracle checks on
sampled heads and sampled batch rows:
  * chunk == per-token recurrence on the layer's own projected inputs (the
    reference's invariant, tests/stable_chunk.rs:11-63), two independent
    kernels on identical operands;
  * the sampled (batch, value head) sequences against the double recurrence
    of the oracle (outputs and final state);
  * token-by-token decode after a prefill == one forward over the whole
    sequence (src/module.rs:224-316; tests/autodiff.rs:31-104);
  * the whole layer (hipBLASLt GEMMs at K = 2048, projection epilogue,
    recurrence, gated norm, o_proj) against the double layer oracle on
    causal prefixes of sampled batch rows, on whole sampled rows for the
    decode configuration, and for the long-context configuration on its last
    256 tokens from the layer's own state at that point.
Tolerance: max |error| <= 1e-4 (tests/test_chunk.rs:254-255); layer outputs
(about 2e-3 in size) also within 1e-4 of max |reference|.
The GVA configuration is checked against true head repeat (value head hv
reads key head hv / rep), not the reference's time-scrambling reshape."""
import numpy as np
import pytest

from gdn2_testutil import maxabs
from oracle import oracle as O

TOL = 1e-4

pytestmark = pytest.mark.gpu


def _layer(G, seed=1337, dt_shift=0.0, **over):
    cfg = G.Gdn2Config(**over)
    layer = G.GatedDeltaNet2(cfg, seed=seed)
    if dt_shift:
        layer.set_param("dt_bias", layer.param("dt_bias") + np.float32(dt_shift))
    return cfg, layer


def _x(torch, gpu, seed, shape):
    gen = torch.Generator(device=gpu)
    gen.manual_seed(seed)
    return torch.randn(shape, generator=gen, device=gpu, dtype=torch.float32)


def _vs_oracle(got, ref, what):
    """max |got - ref| <= 1e-4 and <= 1e-4 max |ref|."""
    got = np.asarray(got, np.float64)
    err = maxabs(got, ref)
    scale = float(np.abs(ref).max())
    print(f"{what}: max|err| {err:.2e}  max|ref| {scale:.3e}  ratio {err / max(scale, 1e-30):.2e}", flush=True)
    assert np.isfinite(got).all(), what
    assert err <= TOL and err <= TOL * scale, (what, err, scale)


def _layer_prefix_vs_oracle(cfg, layer, x, out, rows, T):
    """out[rows, :T] (a causal prefix of forward_train / forward from no
    state) against the double layer oracle on x[rows, :T] with the layer's
    own weights."""
    xr = x[rows, :T].contiguous().cpu().numpy()
    ref, _ = O.layer_forward(cfg, layer.params(), xr)
    _vs_oracle(out[rows, :T].cpu().numpy(), ref.out, f"layer rows {rows} tokens [0, {T}) vs oracle")


def _oracle_state(st, rows):
    return O.OracleState(st.recurrent[rows], st.conv_q[rows], st.conv_k[rows], st.conv_v[rows])


def _core_views(P):
    """project() outputs, already in the reference's [B, H, T, D] layout."""
    return [P[n] for n in ("q", "k", "v", "g", "b", "w")]


def _check_core(G, cfg, P, chunk_size, sample, S0=None):
    """chunk == recurrence on all heads; sampled heads == the double oracle."""
    import torch

    q, k, v, g, b, w = _core_views(P)
    B, HV, K, V = q.shape[0], cfg.hv, cfg.head_dim, cfg.v_head
    scale = K ** -0.5
    S = torch.zeros((B, HV, K, V), device=q.device) if S0 is None else S0
    res = G.chunk_wy_forward(q, k, v, g, b, w, S, scale, chunk_size=chunk_size)
    assert res is not None
    oc, Sc = res
    orr, Sr = G.fused_recurrent_forward(q, k, v, g, b, w, S, scale)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(oc).all()) and bool(torch.isfinite(Sc).all())
    e_o = float((oc - orr).abs().max())
    e_s = float((Sc - Sr).abs().max())
    print(f"chunk vs recurrence: out {e_o:.2e}  S {e_s:.2e}", flush=True)
    assert e_o < TOL and e_s < TOL
    rep = HV // cfg.num_heads
    for bi, hv in sample:
        hk = hv // rep
        hq = [t[bi:bi + 1, hk:hk + 1].contiguous().cpu().numpy() for t in (q, k)]
        hg = [t[bi:bi + 1, hk:hk + 1].contiguous().cpu().numpy() for t in (g, b)]
        hvw = [t[bi:bi + 1, hv:hv + 1].contiguous().cpu().numpy() for t in (v, w)]
        S0h = None if S0 is None else S0[bi:bi + 1, hv:hv + 1].cpu().numpy()
        o_ref, S_ref = O.recurrent_f64(hq[0], hq[1], hvw[0], hg[0], hg[1], hvw[1], S0=S0h, scale=scale)
        eo = maxabs(oc[bi:bi + 1, hv:hv + 1].cpu().numpy(), o_ref)
        es = maxabs(Sc[bi:bi + 1, hv:hv + 1].cpu().numpy(), S_ref)
        print(f"oracle (b={bi}, hv={hv}): out {eo:.2e}  S {es:.2e}", flush=True)
        assert eo < TOL and es < TOL
    return oc, Sc


def test_config2_default_prefill_chunk(gpu):
    """hidden 2048, 16 heads, head_dim 128, chunk 64, x [8, 4096, 2048]."""
    import torch

    import gdn2_amd as G

    cfg, layer = _layer(G, hidden_size=2048, num_heads=16, head_dim=128, mode="chunk", chunk_size=64)
    x = _x(torch, gpu, 42, (8, 4096, 2048))
    P = layer.project(x)
    _check_core(G, cfg, P, 64, sample=[(0, 0), (7, 15), (3, 9)])
    del P
    out = layer.forward_train(x)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())
    _layer_prefix_vs_oracle(cfg, layer, x, out, [0, 7], 512)


def test_config3_decode_reproduces_full_forward(gpu):
    """B = 64: prefill 2048 tokens, then 256 single tokens, against one
    forward over all 2304 tokens (FusedRecurrent mode)."""
    import torch

    import gdn2_amd as G

    cfg, layer = _layer(G, hidden_size=2048, num_heads=16, head_dim=128)
    Bd, Tp, Td = 64, 2048, 256
    x = _x(torch, gpu, 43, (Bd, Tp + Td, 2048))
    full, st_full = layer.forward(x)
    out_p, st = layer.forward(x[:, :Tp].contiguous())
    outs = []
    for t in range(Tp, Tp + Td):
        o, st = layer.forward(x[:, t:t + 1].contiguous(), st)
        outs.append(o)
    dec = torch.cat(outs, 1)
    torch.cuda.synchronize()
    e_pre = float((out_p - full[:, :Tp]).abs().max())
    e_dec = float((dec - full[:, Tp:]).abs().max())
    scale = float(full.abs().max())
    e_s = maxabs(st.recurrent, st_full.recurrent)
    print(f"prefill {e_pre:.2e}  decode {e_dec:.2e} (max|out| {scale:.3e})  S {e_s:.2e}", flush=True)
    assert e_pre < TOL and e_dec < TOL and e_dec <= 1e-4 * scale and e_s < TOL
    for n in ("conv_q", "conv_k", "conv_v"):  # raw projections, up to the GEMMs' rounding at other M
        assert maxabs(getattr(st, n), getattr(st_full, n)) < 1e-5, n
    # whole sampled batch rows against the double layer oracle: the prefill's
    # outputs, the 256 decoded tokens, the final recurrent state and conv caches
    rows = [0, 37]
    ref, rst = O.layer_forward(cfg, layer.params(), x[rows].contiguous().cpu().numpy())
    _vs_oracle(out_p[rows].cpu().numpy(), ref.out[:, :Tp], f"prefill rows {rows} vs oracle")
    _vs_oracle(dec[rows].cpu().numpy(), ref.out[:, Tp:], f"decoded tokens rows {rows} vs oracle")
    e_so = maxabs(st.recurrent[rows], rst.recurrent)
    print(f"final S rows {rows} vs oracle: {e_so:.2e}", flush=True)
    assert e_so < TOL
    for n in ("conv_q", "conv_k", "conv_v"):
        assert maxabs(getattr(st, n)[rows], getattr(rst, n)) < TOL, n
    # the core of the one-pass forward against the double oracle on sampled heads
    P = layer.project(x[:4, :512].contiguous())
    _check_core(G, cfg, P, 64, sample=[(0, 0), (3, 11)])


def test_config4_gva_negeig_mindecay_chunk_then_decode(gpu):
    """hidden 2048, 8 key heads, 16 value heads, head_dim 128, expand_v 2,
    allow_neg_eigval, min_decay 0.9, x [4, 8192, 2048]; then decode."""
    import torch

    import gdn2_amd as G

    cfg, layer = _layer(G, hidden_size=2048, num_heads=8, num_v_heads=16, head_dim=128, expand_v=2.0,
                        allow_neg_eigval=True, min_decay=0.9, mode="chunk")
    B, T, Td = 4, 8192, 32
    x = _x(torch, gpu, 44, (B, T + Td, 2048))
    P = layer.project(x[:, :T].contiguous())
    assert float(P["b"].max()) > 1.0  # erase gates in [0, 2]
    _check_core(G, cfg, P, 64, sample=[(0, 0), (1, 7), (3, 15)])
    del P
    full, st_full = layer.forward(x)
    torch.cuda.synchronize()
    _layer_prefix_vs_oracle(cfg, layer, x, full, [0, 3], 512)
    _, st = layer.forward(x[:, :T].contiguous())
    outs = []
    for t in range(T, T + Td):
        o, st = layer.forward(x[:, t:t + 1].contiguous(), st)
        outs.append(o)
    dec = torch.cat(outs, 1)
    torch.cuda.synchronize()
    e_dec = float((dec - full[:, T:]).abs().max())
    e_s = maxabs(st.recurrent, st_full.recurrent)
    print(f"decode {e_dec:.2e} (max|out| {float(full.abs().max()):.3e})  S {e_s:.2e}", flush=True)
    assert e_dec < TOL and e_s < TOL
    # the 32 decoded tokens of rows 0 and 3 against the double layer oracle
    # started from the layer's own state after the 8192-token prefill (S and
    # the conv caches), token by token like the decode calls
    _, st_p = layer.forward(x[:, :T].contiguous())
    rows = [0, 3]
    ost = _oracle_state(st_p, rows)
    ref, rst = O.layer_forward(cfg, layer.params(), x[rows, T:].contiguous().cpu().numpy(), state=ost)
    _vs_oracle(dec[rows].cpu().numpy(), ref.out, f"32 decoded tokens rows {rows} vs oracle from the prefill state")
    e_so = maxabs(st.recurrent[rows], rst.recurrent)
    print(f"final S rows {rows} vs oracle: {e_so:.2e}", flush=True)
    assert e_so < TOL


def test_config5_long_context_strong_decay(gpu):
    """B = 1, T = 65536, chunk_size 128, dt_bias + 4: cumulative log-decays
    fall far below -88 inside a chunk; outputs and state stay finite and
    match the recurrence."""
    import torch

    import gdn2_amd as G

    cfg, layer = _layer(G, dt_shift=4.0, hidden_size=2048, num_heads=16, head_dim=128, mode="chunk",
                        chunk_size=128)
    x = _x(torch, gpu, 45, (1, 65536, 2048))
    P = layer.project(x)
    g = P["g"]  # [1, H, T, K]
    span = float(-g[0, :, :128].sum(1).min())  # cumulative decay over the first 128-token chunk
    print(f"cumulative log-decay over one chunk reaches -{span:.1f}", flush=True)
    assert span > 88.0
    _check_core(G, cfg, P, 128, sample=[(0, 0), (0, 13)])
    del P
    out = layer.forward_train(x)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())
    _layer_prefix_vs_oracle(cfg, layer, x, out, [0], 512)
    # the last 256 tokens: continued from the layer's own state after the first
    # T - 256 tokens, against forward_train's tail and the double layer oracle
    # started from that same state
    T, t0 = x.shape[1], x.shape[1] - 256
    _, st = layer.forward(x[:, :t0].contiguous())
    st_t0 = _oracle_state(st, [0])  # forward() updates the state object in place
    tail, st_end = layer.forward(x[:, t0:].contiguous(), st)
    torch.cuda.synchronize()
    e_cont = float((tail - out[:, t0:]).abs().max())
    print(f"tail after a {t0}-token prefill vs forward_train: {e_cont:.2e}", flush=True)
    assert e_cont < TOL and e_cont <= TOL * float(out[:, t0:].abs().max())
    ref, rst = O.layer_forward(cfg, layer.params(), x[:, t0:].contiguous().cpu().numpy(), state=st_t0)
    _vs_oracle(tail.cpu().numpy(), ref.out, f"last 256 tokens of {T} vs oracle from the same state")
    e_s = maxabs(st_end.recurrent, rst.recurrent)
    print(f"final S vs oracle: {e_s:.2e}", flush=True)
    assert e_s < TOL

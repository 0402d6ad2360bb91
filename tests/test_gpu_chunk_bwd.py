"""GPU parity of the chunked backward (gdn2_chunk_bwd_f32) against the
oracle's f64 adjoint of the recurrence (itself pinned by finite differences
in test_oracle_bwd.py).  Tolerance per gradient tensor: max |error| <=
1e-4 * max(1, max |reference|) -- f32 kernels against the f64 adjoint over
the whole sequence (the forward's 1e-4 bound, scaled to the gradient's
magnitude, which grows with the sequence)."""
import numpy as np
import pytest

from conftest import rand_inputs
from oracle import oracle as O

pytestmark = pytest.mark.gpu

NAMES = ("dq", "dk", "dg", "db", "dv", "dw", "dS0")


def _dev(gpu, *arrs):
    import torch

    return [torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(gpu) for a in arrs]


def _compare(got, ref, label):
    worst = {}
    for n in NAMES:
        g = got[n].cpu().numpy().astype(np.float64)
        r = ref[n]
        err = float(np.abs(g - r).max()) if r.size else 0.0
        bound = 1e-4 * max(1.0, float(np.abs(r).max()) if r.size else 0.0)
        worst[n] = (err, bound)
    print(label, " ".join(f"{n}={e:.1e}/{b:.0e}" for n, (e, b) in worst.items()))
    for n, (e, b) in worst.items():
        assert e <= b, (label, n, e, b)


CASES = [
    # B, Hk, HV, T, K, V, g range, b_hi, S0 scale, d_state_out
    (1, 1, 1, 64, 128, 128, (-0.3, -0.02), 1.0, 0.5, True),
    (2, 2, 2, 130, 128, 128, (-0.3, -0.02), 1.0, 0.5, True),    # ragged last chunk
    (1, 1, 2, 150, 128, 256, (-0.4, -0.01), 2.0, 0.5, True),    # GVA rep 2, V = 2K, negative eigenvalues
    (2, 2, 2, 97, 64, 64, (-0.3, -0.02), 1.0, 0.0, False),      # K = V = 64, no state gradient in
    (1, 2, 2, 200, 128, 128, (-5.0, -0.5), 1.0, 0.5, True),     # strong decay
    (1, 1, 1, 1, 128, 128, (-0.3, -0.02), 1.0, 1.0, True),      # T = 1
    (1, 1, 2, 63, 64, 128, (-1.0, -0.1), 2.0, 0.3, True),
    (1, 1, 1, 100, 128, 64, (-0.3, -0.02), 1.0, 0.5, True),     # V = K / 2: four value slices
    (1, 1, 1, 90, 64, 256, (-0.5, -0.05), 1.0, 0.5, True),      # V = 4 K: sixteen value slices
    (1, 2, 2, 2100, 128, 128, (-0.003, -0.0005), 1.0, 1.0, True),  # slow decay; seven segments of 5 chunks
    (1, 2, 2, 2560, 128, 128, (-0.001, 0.0), 0.0, 1.0, True),       # b = 0: S0 and d_state carried through
    (1, 1, 2, 6400, 64, 128, (-0.002, 0.0), 2.0, 1.0, True),        # 25 segments, GVA, negative eigenvalues
    # the forward's other head shapes: two-wave reverse-recurrence workgroups (32 value columns)
    (2, 2, 2, 130, 32, 32, (-0.3, -0.02), 1.0, 0.5, True),      # K = V = 32, ragged last chunk
    (1, 1, 2, 150, 32, 64, (-0.5, -0.05), 2.0, 0.5, True),      # K = 32, V = 64, GVA, negative eigenvalues
    (2, 1, 1, 97, 64, 96, (-0.3, -0.02), 1.0, 0.5, True),       # V = 96 (expand_v 1.5)
    (1, 1, 1, 100, 128, 192, (-0.4, -0.01), 1.0, 0.5, False),   # V = 192
    (1, 1, 1, 2100, 64, 96, (-0.003, -0.0005), 1.0, 1.0, True),   # segmented, V = 96
    (1, 1, 2, 3000, 32, 32, (-0.002, 0.0), 2.0, 1.0, True),       # segmented, K = 32, GVA, negative eigenvalues
]


# Decays whose 16-token spans leave the diagonal score blocks' boundary
# reference (spans above 96 in log2 units, in the forward's chunk-intra and the
# backward's decay pass): spans in (96, 192] move the reference to the middle
# of the tile's range; larger ones leave the MFMA product, and the forward
# forms them from half-block products where both 8-token halves span at most
# 192, else (and the backward always) exactly, pair by pair.  |g| up to 31 per
# token (the long-context configuration's decays) reaches both of those;
# U(-6, -2) mixes the two references; U(-14, -0.05) reaches all but the last.
STRONG_CASES = [
    (1, 1, 1, 200, 128, 128, (-31.0, -0.05), 1.0, 0.5, True),
    (1, 2, 2, 130, 64, 64, (-31.0, -0.05), 1.0, 0.5, True),     # K = 64, ragged last chunk
    (1, 1, 2, 150, 128, 256, (-31.0, -0.05), 2.0, 0.5, True),   # GVA rep 2, V = 2K, negative eigenvalues
    (1, 1, 2, 100, 64, 256, (-31.0, -0.05), 1.0, 0.5, True),    # GVA, V = 4K
    (2, 2, 2, 190, 128, 128, (-6.0, -2.0), 1.0, 0.5, True),     # masked and unmasked channels mixed
    (1, 1, 1, 2100, 128, 128, (-6.0, -2.0), 2.0, 1.0, True),    # segmented, negative eigenvalues
    (1, 2, 2, 150, 128, 128, (-14.0, -0.05), 1.0, 0.5, True),   # all three regimes
    (1, 1, 2, 130, 64, 256, (-14.0, -0.05), 2.0, 0.5, True),    # all three, GVA, negative eigenvalues
    (1, 1, 1, 200, 32, 32, (-31.0, -0.05), 1.0, 0.5, True),     # K = 32
    (1, 2, 2, 150, 64, 96, (-31.0, -0.05), 2.0, 0.5, True),     # V = 96, negative eigenvalues
]

def span_regimes(g, T):
    """(tile, channel) pairs by the decay span of the 16-token tile,
    -sum(g) log2(e): at most 96 (boundary reference), in (96, 192] (mid-tile
    reference), above 192 with both 8-token halves at most 192 (half-block
    products) and the rest (exact pairwise terms; the backward's decay pass
    takes every span above 192 pairwise).  Tiles start at multiples of 16,
    since the 64-token chunks do."""
    gt = np.asarray(g, np.float64)
    gt = np.pad(gt, [(0, 0), (0, 0), (0, (-T) % 16), (0, 0)])
    half = -gt.reshape(gt.shape[0], gt.shape[1], -1, 2, 8, gt.shape[3]).sum(4) * np.log2(np.e)
    span, hmax = half.sum(3), half.max(3)
    return (int((span <= 96).sum()), int(((span > 96) & (span <= 192)).sum()),
            int(((span > 192) & (hmax <= 192)).sum()), int(((span > 192) & (hmax > 192)).sum()))


def _run_case(gpu, case):
    import torch

    import gdn2_amd

    B, Hk, HV, T, K, V, (glo, ghi), bhi, s0, dst = case
    rng = np.random.default_rng(3000 + T + K + V)
    q, k, v, g, b, w = rand_inputs(rng, B, Hk, HV, T, K, V, g_lo=glo, g_hi=ghi, b_hi=bhi)
    q *= K ** -0.5 * 4
    S0 = (rng.standard_normal((B, HV, K, V)) * s0).astype(np.float32)
    dO = rng.standard_normal((B, HV, T, V)).astype(np.float32)
    dST = rng.standard_normal((B, HV, K, V)).astype(np.float32) if dst else None
    scale = K ** -0.5
    ref = O.recurrent_bwd_f64(q, k, v, g, b, w, dO, S0=S0, d_ST=dST, scale=scale)
    d = _dev(gpu, q, k, v, g, b, w, S0, dO)
    ds = None if dST is None else _dev(gpu, dST)[0]
    got = gdn2_amd.chunk_wy_backward(*d[:7], d[7], scale, 64, d_state=ds)
    assert got is not None
    torch.cuda.synchronize()
    _compare(got, ref, str(case[:6]))
    return g


@pytest.mark.parametrize("case", CASES, ids=[f"B{c[0]}H{c[1]}HV{c[2]}T{c[3]}K{c[4]}V{c[5]}g{c[6][0]}" for c in CASES])
def test_chunk_bwd_matches_adjoint(gpu, case):
    """Sequences of 2048+ tokens at one or two sequences x heads run the
    segmented forward and reverse recurrences (per-segment transitions)."""
    _run_case(gpu, case)


@pytest.mark.parametrize("case", STRONG_CASES,
                         ids=[f"B{c[0]}H{c[1]}HV{c[2]}T{c[3]}K{c[4]}V{c[5]}g{c[6][0]}" for c in STRONG_CASES])
def test_chunk_bwd_strong_decay(gpu, case):
    """The diagonal blocks' mid-tile reference and exact pairwise terms of the
    training forward's chunk-intra and of the backward's decay pass: each
    case reaches the regimes its decay range is chosen for."""
    g = _run_case(gpu, case)
    lo, mid, split, pair = span_regimes(g, case[3])
    print(f"(tile, channel) spans <= 96: {lo}, (96, 192]: {mid}, half-block: {split}, pairwise: {pair}")
    glo = case[6][0]
    if glo < -20:
        assert split > 0 and pair > 0
    if glo < -10:
        assert split > 0
    if glo > -20:
        assert mid > 0
    if glo > -10:
        assert lo > 0


def test_chunk_bwd_strided_views(gpu):
    """q/k/g/b/v/w and d_out as [B, H, T, D] views of [B, T, H, D] storage:
    the gradients come back in the same layouts."""
    import torch

    import gdn2_amd

    rng = np.random.default_rng(9)
    B, H, T, K, V = 2, 3, 140, 128, 128
    q, k, v, g, b, w = rand_inputs(rng, B, H, H, T, K, V)
    q *= 0.3
    dO = rng.standard_normal((B, H, T, V)).astype(np.float32)
    ref = O.recurrent_bwd_f64(q, k, v, g, b, w, dO, scale=0.2)
    bt = [torch.from_numpy(np.ascontiguousarray(a.transpose(0, 2, 1, 3))).to(gpu) for a in (q, k, v, g, b, w, dO)]
    views = [x.permute(0, 2, 1, 3) for x in bt]
    S0 = torch.zeros((B, H, K, V), device=gpu)
    got = gdn2_amd.chunk_wy_backward(*views[:6], S0, views[6], 0.2)
    assert got is not None
    assert got["dq"].stride() == views[0].stride() and got["dv"].stride() == views[2].stride()
    _compare(got, ref, "strided")


K256_CASES = [
    # head_dim 256 (the reference's fused backward host has no K cap,
    # src/kernel/chunk_adjoint_cube.rs:464-520)
    (1, 2, 2, 150, 256, 256, (-0.3, -0.02), 1.0, 0.5, True),     # ragged last chunk
    (1, 1, 2, 130, 256, 128, (-0.4, -0.01), 2.0, 0.5, True),     # V = 128 (expand_v 0.5), GVA, neg-eig
    (1, 1, 1, 100, 256, 256, (-31.0, -0.05), 1.0, 0.5, True),    # masked diagonal channels
    (1, 1, 2, 2100, 256, 256, (-0.003, -0.0005), 1.0, 1.0, True),  # segmented forward and reverse recurrences
]


@pytest.mark.parametrize("case", K256_CASES, ids=[f"B{c[0]}H{c[1]}HV{c[2]}T{c[3]}K{c[4]}V{c[5]}g{c[6][0]}"
                                                  for c in K256_CASES])
def test_chunk_bwd_head_dim_256(gpu, case):
    """The chunked backward at K = 256: every gradient against the double
    adjoint, and the backward from a saved training forward bit-identical to
    the recomputing one."""
    import torch

    import gdn2_amd

    g = _run_case(gpu, case)
    if case[6][0] < -10:
        _, _, split, pair = span_regimes(g, case[3])
        assert split > 0 and pair > 0
    B, Hk, HV, T, K, V, (glo, ghi), bhi, s0, dst = case
    rng = np.random.default_rng(3000 + T + K + V)
    q, k, v, g, b, w = rand_inputs(rng, B, Hk, HV, T, K, V, g_lo=glo, g_hi=ghi, b_hi=bhi)
    q *= K ** -0.5 * 4
    S0 = (rng.standard_normal((B, HV, K, V)) * s0).astype(np.float32)
    dO = rng.standard_normal((B, HV, T, V)).astype(np.float32)
    d = _dev(gpu, q, k, v, g, b, w, S0, dO)
    out, ST, saved = gdn2_amd.chunk_wy_forward_train(*d[:7], K ** -0.5)
    got = gdn2_amd.chunk_wy_backward(*d[:7], d[7], K ** -0.5, 64, saved=saved)
    rec = gdn2_amd.chunk_wy_backward(*d[:7], d[7], K ** -0.5, 64)
    torch.cuda.synchronize()
    for n in NAMES:
        assert torch.equal(got[n], rec[n]), n


def test_chunk_bwd_empty_sequence(gpu):
    import torch

    import gdn2_amd

    rng = np.random.default_rng(10)
    d = _dev(gpu, *rand_inputs(rng, 1, 1, 1, 0, 128, 128))
    S0 = torch.randn((1, 1, 128, 128), device=gpu)
    dST = torch.randn((1, 1, 128, 128), device=gpu)
    dO = torch.empty((1, 1, 0, 128), device=gpu)
    got = gdn2_amd.chunk_wy_backward(*d, S0, dO, 0.1, d_state=dST)
    assert torch.equal(got["dS0"], dST)


def test_chunk_bwd_scalar_broadcast_gates(gpu):
    """g and b with a last dim of 1: dg and db come back in their shape,
    summed over the channels they were broadcast to."""
    import torch

    import gdn2_amd

    B, Hk, HV, T, K, V = 1, 2, 2, 140, 64, 128
    rng = np.random.default_rng(31)
    q, k, v, g, b, w = rand_inputs(rng, B, Hk, HV, T, K, V, g_lo=-0.4, g_hi=-0.02, b_hi=1.0, gdim=1, bdim=1)
    q *= K ** -0.5 * 4
    S0 = (rng.standard_normal((B, HV, K, V)) * 0.5).astype(np.float32)
    dO = rng.standard_normal((B, HV, T, V)).astype(np.float32)
    dST = rng.standard_normal((B, HV, K, V)).astype(np.float32)
    scale = K ** -0.5
    ref = O.recurrent_bwd_f64(q, k, v, g, b, w, dO, S0=S0, d_ST=dST, scale=scale)
    d = _dev(gpu, q, k, v, g, b, w, S0, dO, dST)
    got = gdn2_amd.chunk_wy_backward(*d[:7], d[7], scale, 64, d_state=d[8])
    torch.cuda.synchronize()
    assert tuple(got["dg"].shape) == (B, Hk, T, 1) and tuple(got["db"].shape) == (B, Hk, T, 1)
    _compare(got, ref, "broadcast g, b")


SAVED_CASES = [
    (2, 2, 2, 130, 128, 128, (-0.3, -0.02)),     # ragged last chunk
    (1, 1, 2, 150, 128, 256, (-31.0, -0.05)),    # GVA, V = 2K, masked diagonal channels
    (1, 2, 2, 2100, 128, 128, (-0.003, -0.0005)),  # segmented: every segment's transition kept
    (2, 2, 2, 97, 64, 64, (-0.3, -0.02)),
    (1, 2, 2, 150, 64, 96, (-0.5, -0.05)),       # V = 96: two-wave workgroups
    (1, 1, 2, 2100, 32, 64, (-0.003, -0.0005)),  # K = 32, segmented, GVA
]


@pytest.mark.parametrize("case", SAVED_CASES, ids=[f"B{c[0]}H{c[1]}HV{c[2]}T{c[3]}K{c[4]}V{c[5]}" for c in SAVED_CASES])
def test_chunk_bwd_from_saved_forward(gpu, case):
    """gdn2_chunk_fwd_train_f32 (the forward keeping the backward's inputs,
    the reference's FusedBackwardInputs) then gdn2_chunk_bwd_saved_f32: the
    forward's output and final state match the double recurrence, and the
    gradients are bit-identical to gdn2_chunk_bwd_f32's (which recomputes
    those quantities) and match the double adjoint."""
    import torch

    import gdn2_amd

    B, Hk, HV, T, K, V, (glo, ghi) = case
    rng = np.random.default_rng(4000 + T + K + V)
    q, k, v, g, b, w = rand_inputs(rng, B, Hk, HV, T, K, V, g_lo=glo, g_hi=ghi, b_hi=2.0)
    q *= K ** -0.5 * 4
    S0 = (rng.standard_normal((B, HV, K, V)) * 0.5).astype(np.float32)
    dO = rng.standard_normal((B, HV, T, V)).astype(np.float32)
    dST = rng.standard_normal((B, HV, K, V)).astype(np.float32)
    scale = K ** -0.5
    d = _dev(gpu, q, k, v, g, b, w, S0, dO, dST)
    res = gdn2_amd.chunk_wy_forward_train(*d[:7], scale)
    assert res is not None
    out, ST, saved = res
    o_ref, S_ref = O.recurrent_f64(q, k, v, g, b, w, S0=S0, scale=scale)
    eo = float(np.abs(out.cpu().numpy() - o_ref).max())
    es = float(np.abs(ST.cpu().numpy() - S_ref).max())
    print(f"training forward: max|out err|={eo:.2e} max|S err|={es:.2e}")
    assert eo < 1e-4 and es < 1e-4
    got = gdn2_amd.chunk_wy_backward(*d[:7], d[7], scale, 64, d_state=d[8], saved=saved)
    rec = gdn2_amd.chunk_wy_backward(*d[:7], d[7], scale, 64, d_state=d[8])
    torch.cuda.synchronize()
    for n in NAMES:
        assert torch.equal(got[n], rec[n]), n
    ref = O.recurrent_bwd_f64(q, k, v, g, b, w, dO, S0=S0, d_ST=dST, scale=scale)
    _compare(got, ref, "saved " + str(case[:6]))

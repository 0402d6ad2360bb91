"""GPU parity of the chunk kernels (chunk-intra + chunk-inter).

Reference points: the double per-token recurrence (ground truth) and the
f32 restatement of chunk_wy_forward (the reference tensor path) where that
one stays finite.  Tolerance: max |error| <= 1e-4 on outputs and the final
state (tests/test_chunk.rs:254-255)."""
import numpy as np
import pytest

from conftest import rand_inputs
from gdn2_testutil import maxabs
from oracle import oracle as O

TOL = 1e-4

pytestmark = pytest.mark.gpu


def _dev(gpu, *arrs):
    import torch

    return [torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(gpu) for a in arrs]


CASES = [
    # B, Hk, HV, T, K, V, g range, b_hi, S0 scale
    (2, 2, 2, 64, 128, 128, (-0.3, -0.02), 1.0, 0.0),
    (1, 2, 2, 130, 128, 128, (-0.15, -0.01), 1.0, 1.0),   # ragged, nonzero S0 (tests/test_chunk.rs:200-256)
    (2, 1, 1, 200, 128, 128, (-5.0, -0.5), 1.0, 0.5),     # strong decay (tests/stable_chunk.rs:70-73)
    (1, 2, 2, 256, 128, 128, (-31.0, -0.05), 1.0, 0.5),   # |g| up to 31: in-tile spans beyond f32 exp range
    (1, 2, 4, 150, 128, 256, (-0.4, -0.01), 2.0, 0.5),    # GVA rep 2, V = 2K, negative eigenvalues
    (2, 2, 2, 97, 64, 64, (-0.3, -0.02), 1.0, 0.5),       # K = V = 64 (config 1 shape)
    (1, 1, 1, 1, 128, 128, (-0.3, -0.02), 1.0, 1.0),      # T = 1
    (1, 1, 2, 63, 64, 128, (-1.0, -0.1), 2.0, 0.3),
    (2, 2, 2, 150, 256, 256, (-0.3, -0.02), 1.0, 0.5),    # K = V = 256 (head_dim 256), ragged
    (1, 1, 2, 200, 256, 128, (-0.4, -0.01), 2.0, 0.5),    # K = 256, V = 128, GVA, negative eigenvalues
    (1, 2, 2, 128, 256, 256, (-31.0, -0.05), 1.0, 0.5),   # K = 256 with spans beyond the f32 exp range
    (1, 2, 2, 100, 128, 64, (-0.3, -0.02), 1.0, 0.5),     # K = 128, V = 64, ragged
    (1, 2, 2, 96, 128, 64, (-31.0, -0.05), 1.0, 0.5),     # V = 64 with spans beyond the f32 exp range
    (1, 1, 2, 130, 64, 256, (-31.0, -0.05), 2.0, 0.5),    # K = 64, V = 256, GVA, neg-eig, the exact diagonal path
    # head shapes of the reference's own benchmarks (tests/bench_cuda.rs:71-72: K = V = 32;
    # tests/bit_exact.rs:224-235: K = 64 with expand_v 1.5, V = 96) and expand_v 1.5 at K = 128
    (2, 2, 2, 150, 32, 32, (-0.3, -0.02), 1.0, 0.5),      # K = V = 32, ragged: two-wave sequential workgroups
    (1, 2, 4, 200, 32, 64, (-0.4, -0.01), 2.0, 0.5),      # K = 32, V = 64, GVA, negative eigenvalues
    (1, 2, 2, 130, 32, 32, (-31.0, -0.05), 1.0, 0.5),     # K = 32 with the exact diagonal path
    (2, 2, 2, 140, 64, 96, (-0.3, -0.02), 1.0, 0.5),      # K = 64, V = 96: three 32-column slices
    (1, 1, 2, 97, 64, 96, (-31.0, -0.05), 2.0, 0.5),      # V = 96, GVA, neg-eig, the exact diagonal path
    (1, 2, 2, 150, 128, 192, (-0.3, -0.02), 1.0, 0.5),    # K = 128, V = 192: three 64-column slices
    (1, 1, 2, 100, 128, 192, (-31.0, -0.05), 2.0, 0.5),   # V = 192, GVA, neg-eig, spans beyond the f32 exp range
]


# Decays whose 16-token spans fall mostly in (96, 192] log2 units: the diagonal
# score blocks' mid-tile reference (the wider ranges also reach the boundary
# reference below 96 and the half-block products above 192)
MID_CASES = [
    (1, 2, 2, 200, 128, 128, (-9.0, -3.0), 1.0, 0.5),
    (1, 2, 2, 256, 128, 128, (-14.0, -0.05), 1.0, 0.5),
    (1, 1, 2, 150, 64, 64, (-9.0, -3.0), 2.0, 0.5),       # GVA, negative eigenvalues
    (1, 2, 2, 130, 256, 256, (-9.0, -3.0), 1.0, 0.5),
    (1, 2, 2, 97, 32, 64, (-14.0, -0.05), 1.0, 0.5),
    (1, 1, 2, 140, 64, 96, (-9.0, -3.0), 2.0, 0.5),
    (1, 2, 2, 130, 128, 192, (-14.0, -0.05), 1.0, 0.5),
]


def span_regimes(g, T):
    """(tile, channel) pairs by the decay span of the 16-token tile,
    -sum(g) log2(e): at most 96 (boundary reference), in (96, 192] (mid-tile
    reference), above 192 with both 8-token halves at most 192 (half-block
    products) and the rest (exact pairwise terms).  Tiles start at multiples
    of 16, since the 64-token chunks do."""
    gt = np.asarray(g, np.float64)
    gt = np.pad(gt, [(0, 0), (0, 0), (0, (-T) % 16), (0, 0)])
    half = -gt.reshape(gt.shape[0], gt.shape[1], -1, 2, 8, gt.shape[3]).sum(4) * np.log2(np.e)
    span, hmax = half.sum(3), half.max(3)
    return (int((span <= 96).sum()), int(((span > 96) & (span <= 192)).sum()),
            int(((span > 192) & (hmax <= 192)).sum()), int(((span > 192) & (hmax > 192)).sum()))


def _check_case(gpu, case):
    import gdn2_amd

    B, Hk, HV, T, K, V, (glo, ghi), bhi, s0 = case
    rng = np.random.default_rng(1000 + T + K + V)
    q, k, v, g, b, w = rand_inputs(rng, B, Hk, HV, T, K, V, g_lo=glo, g_hi=ghi, b_hi=bhi)
    q *= K ** -0.5 * 4  # keep |q| comparable to the module's L2-normalised queries
    S0 = (rng.standard_normal((B, HV, K, V)) * s0).astype(np.float32)
    scale = K ** -0.5
    o_ref, S_ref = O.recurrent_f64(q, k, v, g, b, w, S0=S0, scale=scale)
    d = _dev(gpu, q, k, v, g, b, w, S0)
    res = gdn2_amd.chunk_wy_forward(*d, scale, chunk_size=64)
    assert res is not None
    o, S = res
    eo, es = maxabs(o.cpu().numpy(), o_ref), maxabs(S.cpu().numpy(), S_ref)
    print(f"max|out err|={eo:.2e} max|S err|={es:.2e}")
    assert eo < TOL and es < TOL
    # the reference tensor path (f32 restatement) agrees wherever it is finite
    o32, S32 = O.chunk_wy_f32(q, k, v, g, b, w, S0=S0, scale=scale, chunk_size=64)
    if np.all(np.isfinite(o32)) and np.all(np.isfinite(S32)):
        assert maxabs(o.cpu().numpy(), o32) < TOL and maxabs(S.cpu().numpy(), S32) < TOL
    return g


@pytest.mark.parametrize("case", CASES, ids=[f"B{c[0]}H{c[1]}HV{c[2]}T{c[3]}K{c[4]}V{c[5]}g{c[6][0]}" for c in CASES])
def test_chunk_matches_recurrence(gpu, case):
    g = _check_case(gpu, case)
    if case[6][0] < -20:  # |g| up to 31: half-block products and exact pairwise terms
        lo, mid, split, pair = span_regimes(g, case[3])
        print(f"(tile, channel) half-block: {split}, pairwise: {pair}")
        assert split > 0 and pair > 0


@pytest.mark.parametrize("case", MID_CASES,
                         ids=[f"B{c[0]}H{c[1]}HV{c[2]}T{c[3]}K{c[4]}V{c[5]}g{c[6][0]}" for c in MID_CASES])
def test_chunk_mid_span_diagonal(gpu, case):
    """Diagonal score blocks whose decay spans lie between the boundary
    reference's bound (96) and the exact pairwise path (above 192)."""
    g = _check_case(gpu, case)
    lo, mid, split, pair = span_regimes(g, case[3])
    print(f"(tile, channel) spans <= 96: {lo}, (96, 192]: {mid}, half-block: {split}, pairwise: {pair}")
    assert mid > (lo + mid + split + pair) // 2
    if case[6][0] < -10:  # the wide range reaches the boundary reference and the half-block products
        assert lo > 0 and split > 0


def _base_workspace_bytes(B, HV, T, K, V):
    """Workspace of the per-chunk buffers alone (W, q e^G, U, A_qk, Kd^T, e^G_last)."""
    al = lambda x: (x + 255) // 256 * 256
    n = B * HV * ((T + 63) // 64)
    return sum(al(4 * n * e) for e in (64 * K, 64 * K, 64 * V, 64 * 64, 64 * K, K))


SEG_CASES = [
    # few long sequences: chunk-inter splits each sequence into segments (of at
    # least 4 chunks).  Slow decays keep the transitions P far from 0 over a
    # segment, so that S0 and the chaining both reach the output.
    (1, 2, 2, 2530, 128, 128, (-0.003, -0.0005), 1.0, 1.0),  # 40 chunks, ragged end
    (1, 1, 2, 6400, 64, 128, (-0.002, 0.0), 2.0, 1.0),       # GVA, negative eigenvalues, 100 chunks
    (1, 2, 2, 2100, 128, 128, (-0.3, -0.02), 1.0, 0.5),
    (1, 1, 2, 2530, 256, 256, (-0.003, -0.0005), 1.0, 1.0),  # K = V = 256, segmented
    (1, 2, 2, 2560, 128, 128, (-0.001, 0.0), 0.0, 1.0),      # b = 0: P = diag(exp(G)) ~ 0.3-1, S0 carried whole
    (1, 1, 1, 4100, 128, 256, (-5.0, -0.5), 1.0, 1.0),       # strong decay, V = 2K
    (1, 2, 2, 2530, 32, 32, (-0.003, -0.0005), 1.0, 1.0),    # K = V = 32: 32-column slices of P
    (1, 1, 2, 2600, 64, 96, (-0.002, 0.0), 2.0, 1.0),        # V = 96, GVA, negative eigenvalues
    (1, 1, 1, 2400, 128, 192, (-0.003, -0.0005), 1.0, 1.0),  # V = 192
]


@pytest.mark.parametrize("case", SEG_CASES, ids=[f"B{c[0]}H{c[1]}HV{c[2]}T{c[3]}K{c[4]}V{c[5]}" for c in SEG_CASES])
def test_chunk_segmented_matches_recurrence(gpu, case):
    """Segmented chunk-inter (per-segment transition, chained entering
    states, output pass) == the per-token recurrence, with nonzero S0."""
    import torch

    import gdn2_amd

    B, Hk, HV, T, K, V, (glo, ghi), bhi, s0 = case
    rng = np.random.default_rng(2000 + T + K + V)
    q, k, v, g, b, w = rand_inputs(rng, B, Hk, HV, T, K, V, g_lo=glo, g_hi=ghi, b_hi=bhi)
    q *= K ** -0.5 * 4
    S0 = (rng.standard_normal((B, HV, K, V)) * s0).astype(np.float32)
    scale = K ** -0.5
    o_ref, S_ref = O.recurrent_f64(q, k, v, g, b, w, S0=S0, scale=scale)
    d = _dev(gpu, q, k, v, g, b, w, S0)
    out = torch.empty((B, HV, T, V), device=gpu)
    # the segment buffers are present: the segmented form runs for this shape
    assert gdn2_amd.chunk_workspace_bytes(*d, out, scale, 64) > _base_workspace_bytes(B, HV, T, K, V)
    o, S = gdn2_amd.chunk_wy_forward(*d, scale, chunk_size=64)
    eo, es = maxabs(o.cpu().numpy(), o_ref), maxabs(S.cpu().numpy(), S_ref)
    print(f"max|out err|={eo:.2e} max|S err|={es:.2e}")
    assert eo < TOL and es < TOL


def split_plan(B, HV, T, K, V):
    """The inference forward's chunk-inter plan for a shape, restated from
    chunk.hip (inter_segments, split_segments) so that a case can assert which
    form it reaches: (uniform segment count n, None) or (n, (L0, L)) where the
    split walks segment 0 (L0 chunks) beside pass 1 and the other n segments
    have L chunks (the last fewer)."""
    nwv = 4 if (V % 64 == 0 and K % 64 == 0) else 2
    NC = (T + 63) // 64
    w = B * HV * (V // (16 * nwv))
    n = min(256 // w, NC // 4)
    if n < 2:
        return 1, None
    L = -(-NC // n)
    n = -(-NC // L)
    if n < 2:
        return n, None
    r = 1.1 if (K == 128 and V % 128 == 0) else 0.8
    L0 = int(r * NC / (n + r))
    Ls = -(-(NC - L0) // n)
    if L0 < 16 or Ls < 16 or NC - L0 - (n - 1) * Ls < 1:
        return n, None
    return n, (L0, Ls)


SPLIT_CASES = [
    # few long sequences whose uniform run has at most 8 segments of >= 16
    # chunks: segment 0 is walked with the output from S0 beside pass 1 of the
    # others, whose chain then starts from the state segment 0 left
    (1, 8, 16, 10000, 128, 128, (-0.01, -0.001), 1.0, 1.0),  # the long-context class, GVA, ragged end
    (2, 16, 16, 12000, 64, 64, (-0.3, -0.02), 1.0, 0.5),
    (1, 16, 16, 11000, 64, 96, (-0.002, 0.0), 2.0, 1.0),     # V = 96 (two-wave slices), negative eigenvalues
]


@pytest.mark.parametrize("case", SPLIT_CASES,
                         ids=[f"B{c[0]}H{c[1]}HV{c[2]}T{c[3]}K{c[4]}V{c[5]}" for c in SPLIT_CASES])
def test_chunk_split_first_segment_matches_recurrence(gpu, case):
    """The inference forward's split (segment 0 walked once, with the output,
    beside the other segments' summaries; the chain and output pass over the
    rest) == the per-token recurrence, with nonzero S0."""
    import gdn2_amd

    B, Hk, HV, T, K, V, (glo, ghi), bhi, s0 = case
    n, plan = split_plan(B, HV, T, K, V)
    assert plan is not None, (n, plan)
    print(f"case {case}: uniform segments {n}, split (L0, L) = {plan}", flush=True)
    rng = np.random.default_rng(3000 + T + K + V)
    q, k, v, g, b, w = rand_inputs(rng, B, Hk, HV, T, K, V, g_lo=glo, g_hi=ghi, b_hi=bhi)
    q *= K ** -0.5 * 4
    S0 = (rng.standard_normal((B, HV, K, V)) * s0).astype(np.float32)
    scale = K ** -0.5
    d = _dev(gpu, q, k, v, g, b, w, S0)
    o, S = gdn2_amd.chunk_wy_forward(*d, scale, chunk_size=64)
    o_ref, S_ref = O.recurrent_f64(q, k, v, g, b, w, S0=S0, scale=scale)
    eo, es = maxabs(o.cpu().numpy(), o_ref), maxabs(S.cpu().numpy(), S_ref)
    print(f"  max|out err|={eo:.2e} max|S err|={es:.2e}")
    assert eo < TOL and es < TOL


def test_split_forward_from_two_host_threads(gpu):
    """Two host threads launch the split forward at once, each on a stream of
    its own: the library's second stream and its fork and join events are
    shared per device, so each thread's fork/join sequence must stay whole.
    Each result equals the same call made alone, bit for bit."""
    import threading

    import torch

    import gdn2_amd

    B, Hk, HV, T, K, V = 1, 8, 16, 9000, 128, 128
    assert split_plan(B, HV, T, K, V)[1] is not None
    sets = []
    for seed in (11, 12):
        rng = np.random.default_rng(seed)
        q, k, v, g, b, w = rand_inputs(rng, B, Hk, HV, T, K, V, g_lo=-0.05, g_hi=-0.005)
        S0 = (rng.standard_normal((B, HV, K, V)) * 0.3).astype(np.float32)
        sets.append(_dev(gpu, q, k, v, g, b, w, S0))
    scale = K ** -0.5
    ref = []
    for d in sets:
        o, S = gdn2_amd.chunk_wy_forward(*d, scale, chunk_size=64)
        torch.cuda.synchronize()
        ref.append((o.clone(), S.clone()))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    got, errors = [None, None], []
    start = threading.Barrier(2)

    def run(i):
        try:
            with torch.cuda.stream(streams[i]):
                start.wait()
                for _ in range(3):
                    got[i] = gdn2_amd.chunk_wy_forward(*sets[i], scale, chunk_size=64)
                streams[i].synchronize()
        except Exception as e:  # surfaced below, in the test's own thread
            errors.append(e)

    threads = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for i in range(2):
        assert torch.equal(got[i][0], ref[i][0]) and torch.equal(got[i][1], ref[i][1]), f"thread {i}"


def test_chunk_strided_views_and_in_place_state(gpu):
    """q/k/g/b/v/w as [B, H, T, D] views of [B, T, H, D] storage and out
    written straight into [B, T, HV, V] (no permute copies)."""
    import torch

    import gdn2_amd

    rng = np.random.default_rng(5)
    B, H, T, K, V = 2, 3, 140, 128, 128
    q, k, v, g, b, w = rand_inputs(rng, B, H, H, T, K, V)
    q *= 0.3
    o_ref, S_ref = O.recurrent_f64(q, k, v, g, b, w, scale=0.2)
    bt = [torch.from_numpy(np.ascontiguousarray(a.transpose(0, 2, 1, 3))).to(gpu) for a in (q, k, v, g, b, w)]
    views = [x.permute(0, 2, 1, 3) for x in bt]
    S = torch.zeros((B, H, K, V), device=gpu)
    out = torch.empty((B, T, H, V), device=gpu)
    res = gdn2_amd.chunk_wy_forward(*views, S, 0.2, out=out.permute(0, 2, 1, 3), in_place=True)
    assert res is not None
    assert maxabs(out.permute(0, 2, 1, 3).cpu().numpy(), o_ref) < TOL
    assert maxabs(S.cpu().numpy(), S_ref) < TOL


def test_chunk_continuation_equals_one_pass(gpu):
    """Two calls carrying the state (T1 + T2 tokens) == one call over T1 + T2."""
    import torch

    import gdn2_amd

    rng = np.random.default_rng(6)
    B, H, T, K, V = 1, 2, 300, 128, 128
    q, k, v, g, b, w = rand_inputs(rng, B, H, H, T, K, V)
    q *= 0.3
    d = _dev(gpu, q, k, v, g, b, w)
    S = torch.zeros((B, H, K, V), device=gpu)
    o_full, S_full = gdn2_amd.chunk_wy_forward(*d, S, 0.1)
    cut = 100
    o1, S1 = gdn2_amd.chunk_wy_forward(*[x[:, :, :cut] for x in d], S, 0.1)
    o2, S2 = gdn2_amd.chunk_wy_forward(*[x[:, :, cut:] for x in d], S1, 0.1)
    assert maxabs(torch.cat([o1, o2], 2).cpu().numpy(), o_full.cpu().numpy()) < TOL
    assert maxabs(S2.cpu().numpy(), S_full.cpu().numpy()) < TOL


def test_chunk_not_applicable_outside_instances(gpu):
    """K = 16 is outside the chunk kernels: the reference's `None`."""
    import torch

    import gdn2_amd

    rng = np.random.default_rng(7)
    d = _dev(gpu, *rand_inputs(rng, 1, 1, 1, 20, 16, 8))
    assert gdn2_amd.chunk_wy_forward(*d, torch.zeros((1, 1, 16, 8), device=gpu), 0.25) is None


def test_chunk_empty_sequence_keeps_state(gpu):
    import torch

    import gdn2_amd

    rng = np.random.default_rng(8)
    d = _dev(gpu, *rand_inputs(rng, 1, 1, 1, 0, 128, 128))
    S0 = torch.randn((1, 1, 128, 128), device=gpu)
    o, S = gdn2_amd.chunk_wy_forward(*d, S0, 0.1)
    assert o.shape == (1, 1, 0, 128) and torch.equal(S, S0)


@pytest.mark.parametrize("gdim,bdim", [(1, 1), (1, None), (None, 1)])
def test_scalar_broadcast_gates_and_mixed_layouts(gpu, gdim, bdim):
    """g and b with a last dim of 1 -- one value per head and token, the
    Gated DeltaNet special case (src/forward.rs:149,173,180-182;
    tests/stable_chunk.rs scalar-broadcast cases) -- through the chunk and
    the scan operators, with k in a different layout from q."""
    import gdn2_amd

    B, Hk, HV, T, K, V = 2, 2, 4, 150, 128, 128
    rng = np.random.default_rng(77)
    q, k, v, g, b, w = rand_inputs(rng, B, Hk, HV, T, K, V, g_lo=-0.5, g_hi=-0.01, b_hi=2.0, gdim=gdim, bdim=bdim)
    q *= K ** -0.5 * 4
    S0 = (rng.standard_normal((B, HV, K, V)) * 0.5).astype(np.float32)
    scale = K ** -0.5
    o_ref, S_ref = O.recurrent_f64(q, k, v, g, b, w, S0=S0, scale=scale)
    dq, dk, dv, dg, db, dw, dS0 = _dev(gpu, q, k, v, g, b, w, S0)
    dk = dk.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)  # [B, T, H, K] memory, another layout than q
    for name, res in (("chunk", gdn2_amd.chunk_wy_forward(dq, dk, dv, dg, db, dw, dS0, scale, chunk_size=64)),
                      ("scan", gdn2_amd.fused_recurrent_forward(dq, dk, dv, dg, db, dw, dS0, scale))):
        o, S = res
        eo, es = maxabs(o.cpu().numpy(), o_ref), maxabs(S.cpu().numpy(), S_ref)
        print(f"{name}: max|out err|={eo:.2e} max|S err|={es:.2e}")
        assert eo < TOL and es < TOL


@pytest.mark.parametrize("shape", [(8, 16, 16, 512, 128, 128), (1, 2, 2, 4096, 128, 128)],
                         ids=["one-workgroup-per-CU", "segmented"])
def test_chunk_repeat_is_bit_identical(gpu, shape):
    """chunk-inter orders its global -> LDS copies with vmcnt waits behind
    fence-free barriers, and the backward reuses it for the per-chunk states.
    A missed wait would read a buffer mid-copy and change the result from run
    to run; repeated runs on the same inputs must give the same bits."""
    import torch

    import gdn2_amd

    B, Hk, HV, T, K, V = shape
    rng = np.random.default_rng(4242 + T)
    q, k, v, g, b, w = rand_inputs(rng, B, Hk, HV, T, K, V, g_lo=-0.3, g_hi=-0.02, b_hi=1.0)
    q *= K ** -0.5 * 4
    S0 = (rng.standard_normal((B, HV, K, V)) * 0.5).astype(np.float32)
    dO = rng.standard_normal((B, HV, T, V)).astype(np.float32)
    d = _dev(gpu, q, k, v, g, b, w, S0, dO)
    first = None
    for _ in range(4):
        o, S = gdn2_amd.chunk_wy_forward(*d[:7], K ** -0.5, chunk_size=64)
        got = (o.cpu().numpy(), S.cpu().numpy())
        if first is None:
            first = got
        else:
            assert np.array_equal(got[0], first[0]) and np.array_equal(got[1], first[1])
    grads = []
    for _ in range(2):
        gr = gdn2_amd.chunk_wy_backward(*d[:7], d[7], K ** -0.5, 64)
        torch.cuda.synchronize()
        grads.append({n: t.cpu().numpy() for n, t in gr.items()})
    for n in grads[0]:
        assert np.array_equal(grads[0][n], grads[1][n]), n


STATE_CASES = [
    # B, Hk, HV, T, K, V, chunk_size
    (1, 2, 2, 130, 64, 64, 64),      # ragged last chunk
    (2, 1, 2, 200, 128, 128, 64),    # GVA rep 2
    (1, 2, 2, 2100, 128, 256, 64),   # segmented inter (few long sequences), V = 2K
    (1, 2, 2, 160, 64, 64, 32),      # chunk_size 32, a ragged last 64-token chunk holding one boundary
    (2, 1, 2, 208, 128, 128, 16),    # chunk_size 16, GVA rep 2
    (1, 1, 1, 200, 64, 128, 8),      # chunk_size 8
    (1, 2, 2, 2112, 128, 128, 32),   # chunk_size 32 with the segmented inter
    (1, 1, 2, 192, 256, 256, 16),    # K = V = 256, chunk_size 16
    (1, 2, 2, 240, 128, 128, 48),    # chunk_size 48: boundaries at offsets 48, 32, 16 of the 64-token chunks
    (2, 1, 2, 168, 64, 128, 24),     # chunk_size 24, GVA rep 2, a ragged last 64-token chunk
    (1, 1, 1, 96, 64, 64, 48),       # chunk_size 48: the last 64-token chunk starts no caller chunk
    (1, 2, 2, 2112, 128, 128, 33),   # chunk_size 33 with the segmented inter
    (1, 1, 2, 180, 256, 128, 36),    # K = 256, chunk_size 36
    (1, 2, 2, 192, 64, 96, 48),      # V = 96: the states of a 32-column slice
    (1, 1, 1, 160, 32, 32, 32),      # K = V = 32
]


@pytest.mark.parametrize("case", STATE_CASES,
                         ids=[f"B{c[0]}H{c[1]}HV{c[2]}T{c[3]}K{c[4]}V{c[5]}C{c[6]}" for c in STATE_CASES])
def test_chunk_forward_returns_v_new_and_states(gpu, case):
    """fused_chunk_forward's (out, state, v_new, states), src/kernel/chunk_cube.rs:781-952,
    for chunk size C: states[j] is the oracle recurrence's state after C j
    tokens; row r of v_new[j] is the value the delta rule writes at token
    C j + r, which the oracle's consecutive states give through
    S_t - diag(e^{g_t}) S_{t-1} = k_t v_new_t^T (|k_t| = 1).  C = 64 takes any
    T (rows past T are zero); smaller C divide 64 and T, as the reference
    requires T % C == 0."""
    import gdn2_amd

    B, Hk, HV, T, K, V, Cs = case
    rep = HV // Hk
    rng = np.random.default_rng(5000 + T + K + V + Cs)
    q, k, v, g, b, w = rand_inputs(rng, B, Hk, HV, T, K, V, g_lo=-0.2, g_hi=-0.01, b_hi=1.0)
    q *= K ** -0.5 * 4
    S0 = (rng.standard_normal((B, HV, K, V)) * 0.5).astype(np.float32)
    scale = K ** -0.5
    d = _dev(gpu, q, k, v, g, b, w, S0)
    res = gdn2_amd.chunk_wy_forward(*d, scale, chunk_size=Cs, return_states=True)
    assert res is not None
    o, S, vn, st = (t.cpu().numpy() for t in res)
    NC = (T + Cs - 1) // Cs
    assert vn.shape == (B * HV * NC, Cs, V) and st.shape == (B * HV * NC, K, V)
    o_ref, S_ref = O.recurrent_f64(q, k, v, g, b, w, S0=S0, scale=scale)
    assert maxabs(o, o_ref) < TOL and maxabs(S, S_ref) < TOL
    # the oracle's state after every token
    Ss = [S0.astype(np.float64)]
    for t in range(T):
        sl = lambda a: a[:, :, t:t + 1]
        Ss.append(O.recurrent_f64(*(sl(a) for a in (q, k, v, g, b, w)), S0=Ss[-1], scale=scale)[1])
    st_ref = np.stack([Ss[Cs * n] for n in range(NC)], axis=2)  # [B, HV, NC, K, V]
    e_st = maxabs(st.reshape(B, HV, NC, K, V), st_ref)
    vn_ref = np.zeros((B, HV, NC * Cs, V))
    for t in range(T):
        kt = k[:, :, t].astype(np.float64).repeat(rep, axis=1)             # [B, HV, K]
        gt = np.exp(g[:, :, t].astype(np.float64)).repeat(rep, axis=1)     # [B, HV, K]
        dS = Ss[t + 1] - gt[..., None] * Ss[t]
        vn_ref[:, :, t] = np.einsum("bhk,bhkv->bhv", kt, dS)
    e_vn = maxabs(vn.reshape(B, HV, NC * Cs, V), vn_ref)
    print(f"C={Cs}: states {e_st:.2e}  v_new {e_vn:.2e}", flush=True)
    assert e_st < TOL and e_vn < TOL


def test_chunk_states_refuse_other_chunk_sizes(gpu):
    """Chunk sizes above 64, or that do not divide T, have no per-chunk
    tensors (None, the caller's fallback), as in the reference
    (src/kernel/chunk_cube.rs:795-800)."""
    import gdn2_amd

    rng = np.random.default_rng(77)
    q, k, v, g, b, w = rand_inputs(rng, 1, 1, 1, 96, 64, 64)
    d = _dev(gpu, q, k, v, g, b, w, np.zeros((1, 1, 64, 64), np.float32))
    assert gdn2_amd.chunk_wy_forward(*d, 0.125, chunk_size=48, return_states=True) is not None
    assert gdn2_amd.chunk_wy_forward(*d, 0.125, chunk_size=36, return_states=True) is None  # 96 % 36 != 0
    assert gdn2_amd.chunk_wy_forward(*d, 0.125, chunk_size=64 + 64, return_states=True) is None
    assert gdn2_amd.chunk_wy_forward(*d, 0.125, chunk_size=64, return_states=True) is not None
    d2 = _dev(gpu, *(a[:, :, :90] for a in (q, k, v, g, b, w)), np.zeros((1, 1, 64, 64), np.float32))
    assert gdn2_amd.chunk_wy_forward(*d2, 0.125, chunk_size=32, return_states=True) is None  # 90 % 32 != 0


@pytest.mark.parametrize("shape", [(1, 2, 2, 2048, 128, 128), (1, 8, 16, 9000, 128, 128), (2, 2, 2, 300, 128, 128)],
                         ids=["segmented", "split", "one_segment"])
def test_inter_passes_equal_inter(gpu, shape):
    """gdn2_chunk_inter_pass_f32 1, 2, 3 after gdn2_chunk_intra_f32 equal
    gdn2_chunk_inter_f32 bit for bit (the phase bits of the passes, pass 1
    with the split's segment-0 walk beside it, and pass 3 alone being the
    whole inter phase when there is one segment); gdn2_chunk_segments names
    the uniform segment count; other pass numbers are refused."""
    import ctypes

    import torch

    import gdn2_amd
    from gdn2_amd import _capi as C
    from gdn2_amd.ops import _stream, chunk_args

    B, Hk, HV, T, K, V = shape
    assert (split_plan(B, HV, T, K, V)[1] is not None) == (T == 9000)
    rng = np.random.default_rng(77 + T)
    q, k, v, g, b, w = rand_inputs(rng, B, Hk, HV, T, K, V, g_lo=-0.01, g_hi=-0.001)
    S0 = rng.standard_normal((B, HV, K, V)).astype(np.float32)
    d = _dev(gpu, q, k, v, g, b, w)
    scale = K ** -0.5
    L, stream = C.lib(), _stream()
    results = []
    for by_pass in (False, True):
        st = _dev(gpu, S0)[0]
        out = torch.empty((B, HV, T, V), device=gpu)
        ws = torch.empty(gdn2_amd.chunk_workspace_bytes(*d, st, out, scale, 64), dtype=torch.uint8, device=gpu)
        a = chunk_args(*d, st, out, scale, 64, ws)
        nseg = int(L.gdn2_chunk_segments(ctypes.byref(a)))
        assert (nseg > 1) == (shape[3] >= 2048), nseg
        assert nseg == split_plan(B, HV, T, K, V)[0]
        C.check(L.gdn2_chunk_intra_f32(ctypes.byref(a), stream))
        if by_pass:
            for ps in (1, 2, 3):
                C.check(L.gdn2_chunk_inter_pass_f32(ctypes.byref(a), ps, stream))
            for bad in (0, 4):
                assert L.gdn2_chunk_inter_pass_f32(ctypes.byref(a), bad, stream) == C.GDN2_EINVAL
        else:
            C.check(L.gdn2_chunk_inter_f32(ctypes.byref(a), stream))
        torch.cuda.synchronize()
        results.append((out.cpu(), st.cpu()))
    assert torch.equal(results[0][0], results[1][0]) and torch.equal(results[0][1], results[1][1])
    o_ref, S_ref = O.recurrent_f64(q, k, v, g, b, w, S0=S0, scale=scale)
    assert maxabs(results[1][0].numpy(), o_ref) < TOL and maxabs(results[1][1].numpy(), S_ref) < TOL

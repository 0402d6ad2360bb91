"""The chunked forward and backward under HIP graph capture
(torch.cuda.CUDAGraph on the stream the C ABI receives): gdn2_chunk_fwd_f32
on a caller workspace, gdn2_chunk_fwd_noalloc_f32 on the library's static
scratch, the per-token scan, gdn2_chunk_bwd_f32 and the training pair
gdn2_chunk_fwd_train_f32 + gdn2_chunk_bwd_saved_f32.  Each graph is replayed several times with the program's
own eager work in between (new inputs copied into the captured buffers, the
state reset), and every replay must equal the eager call on the same inputs
bit for bit: the entry points launch kernels only (fills by kernel, no
hipMemsetAsync, no allocation), so a replay runs exactly the eager work."""
import ctypes

import numpy as np
import pytest

from conftest import rand_inputs

pytestmark = pytest.mark.gpu


def _capture(torch, fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()  # first call outside the capture (static scratch address lookup, module load)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


def _sets(rng, n, B, Hk, HV, T, K, V):
    out = []
    for _ in range(n):
        q, k, v, g, b, w = rand_inputs(rng, B, Hk, HV, T, K, V, g_lo=-0.4, g_hi=-0.01)
        S0 = (rng.standard_normal((B, HV, K, V)) * 0.3).astype(np.float32)
        out.append((q, k, v, g, b, w, S0))
    return out


FWD_GRAPH_CASES = [(e, s) for e in ("gdn2_chunk_fwd_f32", "gdn2_chunk_fwd_noalloc_f32")
                   for s in ((2, 2, 2, 200, 128, 128), (1, 1, 2, 2048, 128, 128))]
# the inference split (segment 0 walked on a second stream, forked and joined
# by events, beside pass 1): too large for the no-alloc scratch
FWD_GRAPH_CASES.append(("gdn2_chunk_fwd_f32", (1, 8, 16, 9000, 128, 128)))


@pytest.mark.parametrize("entry,shape", FWD_GRAPH_CASES,
                         ids=[f"{e}-B{s[0]}T{s[3]}" + ("-segmented" if s[3] == 2048 else "-split" if s[3] == 9000 else "")
                              for e, s in FWD_GRAPH_CASES])
def test_chunk_forward_replays_in_a_graph(gpu, entry, shape):
    import torch

    import gdn2_amd as G
    from gdn2_amd import _capi as C
    from gdn2_amd import ops

    B, Hk, HV, T, K, V = shape
    sets = _sets(np.random.default_rng(hash(shape) % 1000 + len(entry)), 2, B, Hk, HV, T, K, V)
    bufs = [torch.empty(a.shape, device=gpu) for a in sets[0][:6]]
    S = torch.empty((B, HV, K, V), device=gpu)
    out = torch.empty((B, HV, T, V), device=gpu)
    need = G.chunk_workspace_bytes(*bufs, S, out, K ** -0.5, 64)
    ws = torch.empty(need, dtype=torch.uint8, device=gpu) if entry == "gdn2_chunk_fwd_f32" else None
    a = ops.chunk_args(*bufs, S, out, K ** -0.5, 64, ws)
    fn_c = getattr(C.lib(), entry)

    def fn():
        C.check(fn_c(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))

    def load(i):
        for buf, arr in zip(bufs, sets[i][:6]):
            buf.copy_(torch.from_numpy(arr))
        S.copy_(torch.from_numpy(sets[i][6]))

    ref = []
    for i in range(2):  # eager results
        load(i)
        fn()
        torch.cuda.synchronize()
        ref.append((out.clone(), S.clone()))
    load(0)
    graph = _capture(torch, fn)
    for rep in range(5):
        i = rep % 2
        load(i)  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref[i][0]) and torch.equal(S, ref[i][1]), f"replay {rep}"


def test_scan_replays_in_a_graph(gpu):
    import torch

    import gdn2_amd as G

    B, Hk, HV, T, K, V = 2, 2, 2, 40, 128, 128
    sets = _sets(np.random.default_rng(21), 2, B, Hk, HV, T, K, V)
    bufs = [torch.empty(a.shape, device=gpu) for a in sets[0][:6]]
    S = torch.empty((B, HV, K, V), device=gpu)
    res = {}

    def fn():
        res["o"], res["S"] = G.fused_recurrent_forward(*bufs, S, K ** -0.5)

    def load(i):
        for buf, arr in zip(bufs, sets[i][:6]):
            buf.copy_(torch.from_numpy(arr))
        S.copy_(torch.from_numpy(sets[i][6]))

    ref = []
    for i in range(2):
        load(i)
        fn()
        torch.cuda.synchronize()
        ref.append((res["o"].clone(), res["S"].clone()))
    load(0)
    graph = _capture(torch, fn)
    for rep in range(4):
        i = rep % 2
        load(i)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(res["o"], ref[i][0]) and torch.equal(res["S"], ref[i][1]), f"replay {rep}"


@pytest.mark.parametrize("shape", [(2, 2, 2, 200, 128, 128), (1, 1, 2, 2100, 64, 96)],
                         ids=["B2T200", "B1T2100-segmented-V96"])
def test_chunk_backward_replays_in_a_graph(gpu, shape):
    """gdn2_chunk_bwd_f32 (recomputing the forward's per-chunk quantities),
    and the pair gdn2_chunk_fwd_train_f32 + gdn2_chunk_bwd_saved_f32, each
    captured once: every replay, with new operands and gradients of the
    output and the final state copied in between, equals the eager call on
    the same inputs bit for bit (the segmented shape takes the two-wave
    reverse-recurrence workgroups and their chain)."""
    import torch

    import gdn2_amd as G

    B, Hk, HV, T, K, V = shape
    rng = np.random.default_rng(sum(shape))
    sets = _sets(rng, 2, B, Hk, HV, T, K, V)
    douts = [(rng.standard_normal((B, HV, T, V)).astype(np.float32),
              rng.standard_normal((B, HV, K, V)).astype(np.float32)) for _ in range(2)]
    bufs = [torch.empty(a.shape, device=gpu) for a in sets[0][:6]]
    S0 = torch.empty((B, HV, K, V), device=gpu)
    dO = torch.empty((B, HV, T, V), device=gpu)
    dST = torch.empty((B, HV, K, V), device=gpu)
    names = ("dq", "dk", "dg", "db", "dv", "dw", "dS0")
    res = {}

    def recompute():
        res["g"] = G.chunk_wy_backward(*bufs, S0, dO, K ** -0.5, 64, d_state=dST)

    def pair():
        out, st, saved = G.chunk_wy_forward_train(*bufs, S0, K ** -0.5)
        res["f"] = (out, st)
        res["g"] = G.chunk_wy_backward(*bufs, S0, dO, K ** -0.5, 64, d_state=dST, saved=saved)

    def load(i):
        for buf, arr in zip(bufs, sets[i][:6]):
            buf.copy_(torch.from_numpy(arr))
        S0.copy_(torch.from_numpy(sets[i][6]))
        dO.copy_(torch.from_numpy(douts[i][0]))
        dST.copy_(torch.from_numpy(douts[i][1]))

    for fn in (recompute, pair):
        ref = []
        for i in range(2):  # eager results
            load(i)
            fn()
            torch.cuda.synchronize()
            ref.append([res["g"][n].clone() for n in names] + [t.clone() for t in res.get("f", ())])
        load(0)
        graph = _capture(torch, fn)
        for rep in range(4):
            i = rep % 2
            load(i)  # eager work between replays
            graph.replay()
            torch.cuda.synchronize()
            got = [res["g"][n] for n in names] + list(res.get("f", ()))
            for n, a, r in zip(names + ("out", "state"), got, ref[i]):
                assert torch.equal(a, r), f"{fn.__name__} replay {rep}: {n}"
        res.clear()

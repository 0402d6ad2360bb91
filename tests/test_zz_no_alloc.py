"""gdn2_chunk_fwd_noalloc_f32 (the chunked forward on the library's static
scratch, for callers that cannot allocate) against gdn2_chunk_fwd_f32 (the
same kernels on a caller workspace), through the C ABI.

Two calls in a row, the second with a smaller input, so that the second runs
on scratch that still holds the first call's contents.  Each must equal the
caller-workspace entry point bit for bit (same kernels, same operands) and
the double recurrence of the oracle within max |error| <= 1e-4
(tests/test_chunk.rs:254-255).  A call that needs more workspace than the
scratch holds is refused with GDN2_EINVAL and writes nothing."""
import ctypes

import numpy as np
import pytest

from conftest import rand_inputs
from gdn2_testutil import maxabs
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _call_noalloc(G, q, k, v, g, b, w, S, out, scale):
    import torch

    from gdn2_amd import _capi as C
    from gdn2_amd import ops

    a = ops.chunk_args(q, k, v, g, b, w, S, out, scale, 64)  # no workspace: the entry point ignores it
    st = C.lib().gdn2_chunk_fwd_noalloc_f32(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    return st


def _case(G, gpu, rng, B, Hk, HV, T, K, V):
    import torch

    from gdn2_amd import _capi as C

    q, k, v, g, b, w = rand_inputs(rng, B, Hk, HV, T, K, V)
    S0 = rng.standard_normal((B, HV, K, V)).astype(np.float32) * 0.1
    d = [torch.from_numpy(x).to(gpu) for x in (q, k, v, g, b, w)]
    S0d = torch.from_numpy(S0).to(gpu)
    scale = K ** -0.5
    print(f"case B={B} Hk={Hk} HV={HV} T={T} K={K} V={V}", flush=True)
    res = G.chunk_wy_forward(*d, S0d, scale, chunk_size=64)  # gdn2_chunk_fwd_f32 on a caller workspace
    assert res is not None
    o_ref, S_ref = res
    S = S0d.clone()
    out = torch.full((B, HV, T, V), float("nan"), device=gpu)
    st = _call_noalloc(G, *d, S, out, scale)
    torch.cuda.synchronize()
    assert st == C.GDN2_OK, C.lib().gdn2_last_error()
    assert torch.equal(out, o_ref) and torch.equal(S, S_ref), "static scratch differs from the caller workspace"
    o64, S64 = O.recurrent_f64(q, k, v, g, b, w, S0=S0, scale=scale)
    eo, es = maxabs(out.cpu().numpy(), o64), maxabs(S.cpu().numpy(), S64)
    print(f"  bit-identical to gdn2_chunk_fwd_f32; vs oracle: out {eo:.2e}  S {es:.2e}", flush=True)
    assert eo < TOL and es < TOL


def test_noalloc_matches_workspace_entry_point_twice(gpu):
    import gdn2_amd as G
    from gdn2_amd import _capi as C

    assert C.lib().gdn2_chunk_noalloc_scratch_bytes() == 64 << 20
    rng = np.random.default_rng(11)
    # first: few long sequences (the segmented inter passes also use the scratch)
    _case(G, gpu, rng, B=1, Hk=2, HV=2, T=4096, K=128, V=128)
    # second, smaller: ragged T, GVA, on scratch still holding the first call's data
    _case(G, gpu, rng, B=2, Hk=1, HV=2, T=300, K=128, V=64)


def test_noalloc_refuses_calls_beyond_the_scratch(gpu):
    import torch

    from gdn2_amd import _capi as C
    from gdn2_amd import ops

    B, H, T, K, V = 2, 8, 4096, 128, 128  # 1024 chunks, ~150 MB of workspace
    x = torch.zeros((B, H, T, K), device=gpu)
    S = torch.zeros((B, H, K, V), device=gpu)
    out = torch.full((B, H, T, V), 7.0, device=gpu)
    a = ops.chunk_args(x, x, x, x, x, x, S, out, K ** -0.5, 64)
    need = C.lib().gdn2_chunk_workspace_bytes(ctypes.byref(a))
    assert need > C.lib().gdn2_chunk_noalloc_scratch_bytes()
    st = C.lib().gdn2_chunk_fwd_noalloc_f32(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == C.GDN2_EINVAL
    assert b"static scratch" in C.lib().gdn2_last_error()
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())

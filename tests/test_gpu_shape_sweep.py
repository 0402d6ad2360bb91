"""A seeded sweep over every head shape of the chunk kernels: for each
(K, V) pair, cases drawn from one generator (batch, GVA repeat, T from 1 to
300 with ragged last chunks, decays from slow to spans past 2^192 per
16-token tile, b up to 2 for negative eigenvalues, S0 and d_state_out on or
off).  Each case runs the training forward (gdn2_chunk_fwd_train_f32), the
recomputing backward (gdn2_chunk_bwd_f32) and the backward from the saved
forward (gdn2_chunk_bwd_saved_f32), against the oracle's f64 recurrence and
its f64 adjoint (pinned by finite differences in test_oracle_bwd.py).
Bounds: the forward 1e-4 absolute on the output and the final state
(tests/test_chunk.rs:254-255), the gradients 1e-4 * max(1, max |reference|)
per tensor (test_gpu_chunk_bwd.py's), and the two backwards bit-identical.
dg alone is held to 1e-4 of the larger of its own magnitude and that of the
terms it adds up, max |k * dk|: every term carries a decay factor
exp(G_r - G_s) whose exponent is a difference of f32 cumulative sums of g
within the chunk, as in the reference (src/forward.rs:104-108).  With |g| up
to 31 per token |G| nears 2000 (log2 units) by a chunk's end, where the f32
spacing is 1.2e-4, so those terms carry relative errors near 1e-4 in any
kernel that forms them from such sums; dg, a sum of such terms (|k * dk| up
to ~5 here) that nearly cancel (|dg| ~ 1), would meet a bound on its own
magnitude only by a few percent, or not, in the strongest cases.
GDN2_SWEEP_CASES (default 50, 600 cases in about 10 s) sets the cases per
shape for a deeper run; the cases are seeded, so a deeper run repeats these
and adds more."""
import os

import numpy as np
import pytest

from conftest import rand_inputs
from gdn2_testutil import maxabs
from oracle import oracle as O

pytestmark = pytest.mark.gpu

SHAPES = [(32, 32), (32, 64), (64, 64), (64, 96), (64, 128), (64, 256), (128, 64), (128, 128), (128, 192),
          (128, 256), (256, 128), (256, 256)]
DECAYS = [(-0.3, -0.02), (-1.0, -0.1), (-6.0, -2.0), (-14.0, -0.05), (-31.0, -0.05)]
NAMES = ("dq", "dk", "dg", "db", "dv", "dw", "dS0")


def _draw(K, V, i):
    """Case i of shape (K, V): sizes kept small enough for the f64 oracle
    (about 10^8 multiply-adds per case at K = V = 256)."""
    rng = np.random.default_rng(7000 + 31 * K + V + 1000 * i)
    rep = int(rng.choice([1, 2]))
    Hk = 1 if K * V >= 128 * 256 else int(rng.choice([1, 2]))
    B = int(rng.choice([1, 2]))
    T = int(rng.choice([1, 17, 64, 97, 130, 200, 300]))
    glo, ghi = DECAYS[int(rng.integers(len(DECAYS)))]
    return dict(B=B, Hk=Hk, HV=Hk * rep, T=T, g=(glo, ghi), b_hi=float(rng.choice([1.0, 2.0])),
                s0=float(rng.choice([0.0, 0.5])), dst=bool(rng.integers(2)), seed=int(rng.integers(1 << 30)))


# cases per shape: 50 by default; GDN2_SWEEP_CASES sets it
NCASES = int(os.environ.get("GDN2_SWEEP_CASES", "50"))
CASES = [(K, V, i) for K, V in SHAPES for i in range(NCASES)]


@pytest.mark.parametrize("K,V,i", CASES, ids=[f"K{K}V{V}-{i}" for K, V, i in CASES])
def test_shape_sweep_forward_and_backward(gpu, K, V, i):
    import torch

    import gdn2_amd

    c = _draw(K, V, i)
    print(f"K={K} V={V} case {i}: {c}", flush=True)
    rng = np.random.default_rng(c["seed"])
    q, k, v, g, b, w = rand_inputs(rng, c["B"], c["Hk"], c["HV"], c["T"], K, V, g_lo=c["g"][0], g_hi=c["g"][1],
                                   b_hi=c["b_hi"])
    q *= K ** -0.5 * 4
    S0 = (rng.standard_normal((c["B"], c["HV"], K, V)) * c["s0"]).astype(np.float32)
    dO = rng.standard_normal((c["B"], c["HV"], c["T"], V)).astype(np.float32)
    dST = rng.standard_normal((c["B"], c["HV"], K, V)).astype(np.float32) if c["dst"] else None
    scale = K ** -0.5
    dev = [torch.from_numpy(np.ascontiguousarray(a)).to(gpu) for a in (q, k, v, g, b, w, S0, dO)]
    ds = None if dST is None else torch.from_numpy(dST).to(gpu)

    res = gdn2_amd.chunk_wy_forward_train(*dev[:7], scale)
    assert res is not None
    out, ST, saved = res
    o_ref, S_ref = O.recurrent_f64(q, k, v, g, b, w, S0=S0, scale=scale)
    eo, es = maxabs(out.cpu().numpy(), o_ref), maxabs(ST.cpu().numpy(), S_ref)
    print(f"  training forward: max|out err|={eo:.2e} max|S err|={es:.2e}")
    assert eo < 1e-4 and es < 1e-4

    got = gdn2_amd.chunk_wy_backward(*dev[:7], dev[7], scale, 64, d_state=ds, saved=saved)
    rec = gdn2_amd.chunk_wy_backward(*dev[:7], dev[7], scale, 64, d_state=ds)
    assert got is not None and rec is not None
    torch.cuda.synchronize()
    for n in NAMES:
        assert torch.equal(got[n], rec[n]), n
    ref = O.recurrent_bwd_f64(q, k, v, g, b, w, dO, S0=S0, d_ST=dST, scale=scale)
    term = float(np.abs(k.astype(np.float64) * ref["dk"]).max()) if k.size else 0.0
    for n in NAMES:
        r = ref[n]
        e = float(np.abs(got[n].cpu().numpy().astype(np.float64) - r).max()) if r.size else 0.0
        bound = 1e-4 * max(1.0, float(np.abs(r).max()) if r.size else 0.0, term if n == "dg" else 0.0)
        print(f"  {n}: {e:.1e} / {bound:.0e}")
        assert e <= bound, n

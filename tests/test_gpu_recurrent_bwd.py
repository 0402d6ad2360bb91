"""GPU parity of the scan's backward (gdn2_recurrent_bwd_f32), the adjoint
for head shapes outside the chunked backward's, against the oracle's f64
adjoint of the recurrence (pinned by finite differences in
test_oracle_bwd.py).  Tolerance per gradient tensor as the chunked
backward's: max |error| <= 1e-4 * max(1, max |reference|)."""
import numpy as np
import pytest

from conftest import rand_inputs
from oracle import oracle as O

pytestmark = pytest.mark.gpu

NAMES = ("dq", "dk", "dg", "db", "dv", "dw", "dS0")


def _dev(gpu, *arrs):
    import torch

    return [None if a is None else torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(gpu) for a in arrs]


def _compare(got, ref, label):
    for n in NAMES:
        g = got[n].cpu().numpy().astype(np.float64)
        r = ref[n]
        err = float(np.abs(g - r).max()) if r.size else 0.0
        bound = 1e-4 * max(1.0, float(np.abs(r).max()) if r.size else 0.0)
        print(f"{label} {n} {err:.1e}/{bound:.0e}")
        assert err <= bound, (label, n, err, bound)


CASES = [
    # B, Hk, HV, T, K, V, S0, d_state_out, gdim, bdim
    (2, 2, 2, 70, 16, 24, True, True, None, None),     # the reference's small test heads; two checkpoint segments
    (1, 1, 3, 130, 32, 16, True, False, None, None),   # GVA rep 3, three segments
    (1, 2, 2, 65, 128, 128, False, True, None, None),  # K = V = 128 (the chunk shapes also run here)
    (1, 1, 1, 64, 64, 256, True, True, None, None),    # one full segment, V = 256
    (2, 2, 4, 1, 8, 8, True, True, None, None),        # T = 1
    (1, 2, 2, 40, 16, 16, True, True, 1, 1),           # per-head scalar g and b
]


@pytest.mark.parametrize("case", CASES, ids=[f"B{c[0]}H{c[1]}HV{c[2]}T{c[3]}K{c[4]}V{c[5]}" for c in CASES])
def test_scan_bwd_matches_adjoint(gpu, case):
    import torch

    import gdn2_amd

    B, Hk, HV, T, K, V, s0, dst, gdim, bdim = case
    rng = np.random.default_rng(4000 + T + K + V)
    q, k, v, g, b, w = rand_inputs(rng, B, Hk, HV, T, K, V, g_lo=-0.5, g_hi=-0.02, b_hi=2.0, gdim=gdim, bdim=bdim)
    q *= K ** -0.5 * 4
    S0 = (rng.standard_normal((B, HV, K, V)) * 0.5).astype(np.float32) if s0 else None
    dO = rng.standard_normal((B, HV, T, V)).astype(np.float32)
    dST = rng.standard_normal((B, HV, K, V)).astype(np.float32) if dst else None
    scale = K ** -0.5
    ref = O.recurrent_bwd_f64(q, k, v, g, b, w, dO, S0=S0, d_ST=dST, scale=scale)
    d = _dev(gpu, q, k, v, g, b, w, S0, dO, dST)
    got = gdn2_amd.fused_recurrent_backward(*d[:7], d[7], scale, d_state=d[8])
    assert got is not None
    torch.cuda.synchronize()
    _compare(got, ref, str(case[:6]))


def test_scan_bwd_empty_sequence_and_limits(gpu):
    import torch

    import gdn2_amd

    rng = np.random.default_rng(5)
    q, k, v, g, b, w = rand_inputs(rng, 1, 1, 1, 0, 16, 16)
    dST = rng.standard_normal((1, 1, 16, 16)).astype(np.float32)
    d = _dev(gpu, q, k, v, g, b, w, None, np.zeros((1, 1, 0, 16), np.float32), dST)
    got = gdn2_amd.fused_recurrent_backward(*d[:7], d[7], 0.25, d_state=d[8])
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got["dS0"].cpu().numpy(), dST)
    # K = V = 256 needs 526 KB of LDS: not this kernel's shape
    q, k, v, g, b, w = rand_inputs(rng, 1, 1, 1, 4, 256, 256)
    d = _dev(gpu, q, k, v, g, b, w, None, np.zeros((1, 1, 4, 256), np.float32))
    assert gdn2_amd.fused_recurrent_backward(*d[:7], d[7], 0.06) is None

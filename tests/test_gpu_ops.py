"""The reference's standalone operators through the C ABI (src/lib.rs:58-62):
short_conv_1d, l2_normalize(_4d) and rms_norm_gate_per_head, against the
oracle's restatements (double) on the same f32 inputs.  Tolerance: max |error|
<= 1e-5 relative to max |reference| (single elementwise passes in f32)."""
import numpy as np
import pytest

from gdn2_testutil import maxabs
from oracle import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _t(gpu, a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(gpu)


@pytest.mark.parametrize("B,T,C,cache", [(2, 1, 96, False), (2, 2, 96, True), (1, 130, 300, False),
                                         (3, 200, 2048, True), (1, 0, 64, True)])
def test_short_conv_matches_oracle(gpu, B, T, C, cache):
    """Replicate padding without a cache, continuation with one, T < 3
    (the new cache still holds cache rows), T = 0 (the cache passes through)."""
    import gdn2_amd as G

    rng = np.random.default_rng(B * 1000 + T + C)
    x = rng.standard_normal((B, T, C)).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, (C, 4)).astype(np.float32)
    c0 = rng.standard_normal((B, 3, C)).astype(np.float32) if cache else None
    y, nc = G.short_conv_1d(_t(gpu, x), _t(gpu, w), None if c0 is None else _t(gpu, c0))
    y_ref, nc_ref = O.short_conv(x, w, c0)
    assert y.shape == (B, T, C) and nc.shape == (B, 3, C)
    if T:
        assert maxabs(y.cpu().numpy(), y_ref) <= TOL * max(1.0, float(np.abs(y_ref).max()))
    assert maxabs(nc.cpu().numpy(), nc_ref) == 0.0  # the cache is a copy of inputs


def test_short_conv_continues_a_sequence(gpu):
    """Token by token with the returned cache equals one pass
    (src/short_conv.rs:13-17)."""
    import torch

    import gdn2_amd as G

    rng = np.random.default_rng(3)
    x = _t(gpu, rng.standard_normal((2, 9, 40)))
    w = _t(gpu, rng.uniform(-0.5, 0.5, (40, 4)))
    full, c_full = G.short_conv_1d(x, w)
    y, c = G.short_conv_1d(x[:, :4].contiguous(), w)
    parts = [y]
    for t in range(4, 9):
        y, c = G.short_conv_1d(x[:, t:t + 1].contiguous(), w, c)
        parts.append(y)
    torch.cuda.synchronize()
    assert float((torch.cat(parts, 1) - full).abs().max()) <= 1e-6
    assert torch.equal(c, c_full)


@pytest.mark.parametrize("shape", [(5, 7), (2, 3, 4, 128), (1, 2, 300, 64), (4, 1000)])
def test_l2_normalize_matches_oracle(gpu, shape):
    import gdn2_amd as G

    rng = np.random.default_rng(len(shape) * 100 + shape[-1])
    x = rng.standard_normal(shape).astype(np.float32)
    x[..., 0, :] *= 1e-4 if len(shape) > 1 else 1.0  # rows where eps matters
    y = G.l2_normalize(_t(gpu, x), 1e-6).cpu().numpy()
    assert maxabs(y, O.l2norm(x, 1e-6)) <= TOL


@pytest.mark.parametrize("shape", [(2, 5, 3, 64), (1, 300, 16, 128), (1, 1, 2, 256)])
def test_rms_norm_gate_matches_oracle(gpu, shape):
    import gdn2_amd as G

    rng = np.random.default_rng(shape[1] + shape[3])
    x = rng.standard_normal(shape).astype(np.float32)
    gate = (rng.standard_normal(shape) * 3).astype(np.float32)
    wn = rng.uniform(0.5, 1.5, shape[-1]).astype(np.float32)
    y = G.rms_norm_gate_per_head(_t(gpu, x), _t(gpu, gate), _t(gpu, wn), 1e-5).cpu().numpy()
    ref = O.rmsnorm_gate(x, gate, wn, 1e-5)
    assert maxabs(y, ref) <= TOL * float(np.abs(ref).max())


def test_ops_refuse_bad_arguments(gpu):
    import torch

    import gdn2_amd as G
    from gdn2_amd import _capi as C

    x = torch.zeros((1, 0, 8), device=gpu)
    w = torch.zeros((8, 4), device=gpu)
    with pytest.raises(C.Gdn2Error):
        G.short_conv_1d(x, w)  # no tokens and no cache
    with pytest.raises(ValueError):
        G.short_conv_1d(torch.zeros((1, 4, 8), device=gpu), torch.zeros((8, 3), device=gpu))
    # in-place use: the conv's tiles read rows that other tiles overwrite
    xs = torch.zeros((2, 100, 8), device=gpu)
    cache = torch.zeros((2, 3, 8), device=gpu)
    lib = C.lib()
    st = lib.gdn2_short_conv_f32(xs.data_ptr(), w.data_ptr(), None, xs.data_ptr(), cache.data_ptr(), 2, 100, 8, None)
    assert st == C.GDN2_EINVAL and "overlap" in lib.gdn2_last_error().decode()
    # a disjoint out is accepted
    out = torch.empty_like(xs)
    assert lib.gdn2_short_conv_f32(xs.data_ptr(), w.data_ptr(), None, out.data_ptr(), cache.data_ptr(), 2, 100, 8,
                                   None) == C.GDN2_OK
    torch.cuda.synchronize()

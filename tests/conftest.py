import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "burn-gdn2_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libgdn2_amd.so")


@pytest.fixture(scope="session")
def gpu():
    """torch with a visible gfx950 device; the GPU tests never fall back."""
    import torch

    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    import gdn2_amd

    assert gdn2_amd.hip_available(), "libgdn2_amd.so reports no usable gfx950 device"
    return torch.device("cuda:0")


def rand_inputs(rng, B, Hk, HV, T, K, V, g_lo=-0.3, g_hi=-0.02, b_hi=1.0, gdim=None, bdim=None):
    """Kernel-level inputs following tests/stable_chunk.rs:15-25: q ~ N(0,1),
    L2-normalised k, v, w ~ N(0,1), g ~ U(g_lo, g_hi), b ~ U(0, b_hi)."""
    gdim = K if gdim is None else gdim
    bdim = K if bdim is None else bdim
    q = rng.standard_normal((B, Hk, T, K)).astype(np.float32)
    kr = rng.standard_normal((B, Hk, T, K))
    k = (kr / np.sqrt((kr * kr).sum(-1, keepdims=True))).astype(np.float32)
    v = rng.standard_normal((B, HV, T, V)).astype(np.float32)
    w = rng.standard_normal((B, HV, T, V)).astype(np.float32)
    g = rng.uniform(g_lo, g_hi, (B, Hk, T, gdim)).astype(np.float32)
    b = rng.uniform(0.0, b_hi, (B, Hk, T, bdim)).astype(np.float32)
    return q, k, v, g, b, w

"""gdn2_stream_copy_f32, the streaming copy behind the benchmark's practical
HBM roof: copies exactly (any length, any grid size) and refuses misaligned
pointers without touching the destination."""
import ctypes

import pytest

pytestmark = pytest.mark.gpu


def _copy(dst, src, n, wg):
    import torch

    from gdn2_amd import _capi as C

    return C.lib().gdn2_stream_copy_f32(ctypes.c_void_p(dst.data_ptr()), ctypes.c_void_p(src.data_ptr()), n, wg,
                                        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


@pytest.mark.parametrize("n,wg", [(1, 0), (3, 0), (4, 1), (1027, 3), (1 << 20, 0), ((1 << 22) + 5, 64)])
def test_stream_copy_is_exact(gpu, n, wg):
    import torch

    from gdn2_amd import _capi as C

    src = torch.randn(n + 8, device=gpu)
    dst = torch.full_like(src, 7.0)
    assert _copy(dst, src, n, wg) == C.GDN2_OK
    torch.cuda.synchronize()
    assert torch.equal(dst[:n], src[:n])
    assert bool((dst[n:] == 7.0).all())  # nothing past n


def test_stream_copy_refuses_misaligned(gpu):
    import torch

    from gdn2_amd import _capi as C

    src = torch.randn(64, device=gpu)
    dst = torch.full_like(src, 7.0)
    assert _copy(dst[1:], src, 16, 0) == C.GDN2_EINVAL
    torch.cuda.synchronize()
    assert bool((dst == 7.0).all())

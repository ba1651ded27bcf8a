"""flashrnn() front-end behaviour on the GPU: mixed input dtypes."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_mixed_dtypes_promote_to_fp32():
    """BF16 Wx with FP32 R and b runs as the all-FP32 call (same bits), the history comes
    back in Wx's dtype and every gradient in its input's dtype."""
    from flashrnn_amd import flashrnn, set_strict

    set_strict(True)
    g = torch.Generator().manual_seed(11)
    B, T, N, D = 5, 12, 2, 64
    wx = torch.randn(B, T, 4, N, D, generator=g).bfloat16().cuda()
    R = (torch.randn(4, N, D, D, generator=g) / D**0.5).cuda()
    b = (0.1 * torch.randn(4, N, D, generator=g)).cuda()
    s0 = torch.randn(2, B, 1, N, D, generator=g).cuda()
    mixed = [wx.clone().requires_grad_(), R.clone().requires_grad_(), b.clone().requires_grad_(),
             s0.clone().requires_grad_()]
    full = [wx.float().requires_grad_(), R.clone().requires_grad_(), b.clone().requires_grad_(),
            s0.clone().requires_grad_()]
    hm, lm = flashrnn(*mixed, function="lstm", dtype="bfloat16")
    hf, lf = flashrnn(*full, function="lstm", dtype="bfloat16")
    assert hm.dtype == torch.bfloat16 and lm.dtype == torch.float32
    torch.testing.assert_close(hm, hf.bfloat16(), atol=0, rtol=0)
    torch.testing.assert_close(lm, lf, atol=0, rtol=0)
    gm = torch.autograd.grad(hm.float().sum() + lm.sum(), mixed)
    gf = torch.autograd.grad(hf.bfloat16().float().sum() + lf.sum(), full)
    for a, e, x in zip(gm, gf, mixed):
        assert a.dtype == x.dtype
        torch.testing.assert_close(a, e.to(x.dtype), atol=0, rtol=0)

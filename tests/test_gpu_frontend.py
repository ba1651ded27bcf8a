"""flashrnn() front-end behaviour on the GPU: mixed input dtypes, the config's layouts and initial_val."""

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


@pytest.mark.parametrize("cell", ["lstm", "gru"])
def test_reference_layouts_and_initial_val(cell):
    """The config's caller-side layouts (input_shape, output_shape, recurrent_shape,
    bias_shape: flashrnn/flashrnn/flashrnn.py:162-170) give the default call's
    results and gradients, permuted, bit for bit; initial_val with states=None
    equals an explicit initial state of that value."""
    from flashrnn_amd import FlashRNNConfig, flashrnn, set_strict
    from tests.test_gpu_parity import make

    set_strict(True)
    cpu, dh, dl = make(cell, 5, 7, 2, 64, seed=41)
    base = [t.cuda().bfloat16().requires_grad_() for t in cpu]
    h, l = flashrnn(*base, function=cell)
    g = torch.autograd.grad((h.float() * dh.cuda()).sum() + (l.float() * dl.cuda()).sum(), base)

    def to(x, src, dst):
        return x.permute(tuple(src.index(c) for c in dst))

    cfg = FlashRNNConfig(function=cell, input_shape="TBGHD", output_shape="STBHD", recurrent_shape="HPGD",
                         bias_shape="HDG")
    lay = [to(cpu[0], "BTGHD", "TBGHD"), to(cpu[1], "GHDP", "HPGD"), to(cpu[2], "GHD", "HDG"),
           to(cpu[3], "SBTHD", "STBHD")]
    lay = [t.contiguous().cuda().bfloat16().requires_grad_() for t in lay]
    h2, l2 = flashrnn(*lay, config=cfg)
    assert torch.equal(h2, to(h, "SBTHD", "STBHD")) and torch.equal(l2, to(l, "SBTHD", "STBHD"))
    g2 = torch.autograd.grad((h2.float() * to(dh, "SBTHD", "STBHD").cuda()).sum()
                             + (l2.float() * to(dl, "SBTHD", "STBHD").cuda()).sum(), lay)
    for a, e, (src, dst) in zip(g2, g, (("BTGHD", "TBGHD"), ("GHDP", "HPGD"), ("GHD", "HDG"), ("SBTHD", "STBHD"))):
        assert torch.equal(a, to(e, src, dst))

    S = cpu[3].shape[0]
    vals = [0.25 * (k + 1) for k in range(S)]
    h3, l3 = flashrnn(*base[:3], None, config=FlashRNNConfig(function=cell, initial_val=vals))
    s0 = torch.tensor(vals).view(S, 1, 1, 1, 1).expand(cpu[3].shape).cuda().bfloat16()
    h4, l4 = flashrnn(*base[:3], s0, function=cell)
    torch.cuda.synchronize()
    assert torch.equal(h3, h4) and torch.equal(l3, l4)

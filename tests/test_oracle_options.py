"""Pins the oracle of the fused backend's cut / clip options (CPU only).

The reference holds no numeric vectors for ``gradient_recurrent_cut`` and
``gradient_recurrent_clipval`` (they exist only in its CUDA fused/alternating
kernels), so ``oracle.torch_restatement.flashrnn_torch_fused_options`` is
pinned by what the mathematics fixes:

* no option set == ``flashrnn_torch`` bitwise; a clip value no value reaches ==
  no clip; the cut at T=1 == no cut except the initial hidden state's cotangent;
* closed forms: Elman with the cut, dWx_t = dh_t (1 - h_t^2) for any R; the
  straight-through forward clamp, dWx = dh (1 - tanh^2 x) for a clamped step;
  the clamp of GRU's direct path at R = 0 (and none on the initial state's cotangent);
* the forward bound |h| <= v at every step and in the carry;
* two mechanisms that must agree: for cells whose hidden state has no direct
  path (LSTM, sLSTM, Elman) a vanishing clip of the recurrent cotangent equals
  the cut.
"""

import pytest
import torch

from oracle.torch_restatement import SIZES, flashrnn_torch, flashrnn_torch_fused_options
from tests.test_oracle import rand_inputs


def run(fn, leaves, cell, seed=7, **kw):
    g = torch.Generator().manual_seed(seed)
    hist, last = fn(*leaves, cell=cell, **kw)
    dh = torch.randn(hist.shape, generator=g, dtype=hist.dtype)
    dl = torch.randn(last.shape, generator=g, dtype=last.dtype)
    grads = torch.autograd.grad((hist * dh).sum() + (last * dl).sum(), leaves, allow_unused=True)
    grads = [torch.zeros_like(x) if gr is None else gr for gr, x in zip(grads, leaves)]  # unused: zero
    return (hist.detach(), last.detach(), *grads), dh


@pytest.mark.parametrize("cell", list(SIZES))
@pytest.mark.parametrize("numerics", ["mathematical", "fp32_state_bf16_mma"])
def test_no_option_equals_flashrnn_torch(cell, numerics):
    dt = torch.float64 if numerics == "mathematical" else torch.float32
    leaves = rand_inputs(cell, dtype=dt)
    a, _ = run(flashrnn_torch_fused_options, leaves, cell, numerics=numerics)
    e, _ = run(flashrnn_torch, leaves, cell, numerics=numerics)
    for x, y in zip(a, e):
        torch.testing.assert_close(x, y, atol=0, rtol=0)


@pytest.mark.parametrize("cell", list(SIZES))
def test_unreached_clip_is_no_clip(cell):
    # FP64; not bitwise for GRU only: wrapping h_{t-1} changes the order in
    # which autograd sums its two uses (the product and u * h)
    leaves = rand_inputs(cell)
    a, _ = run(flashrnn_torch_fused_options, leaves, cell, gradient_recurrent_clipval=1e30)
    e, _ = run(flashrnn_torch, leaves, cell)
    tol = 1e-13 if cell == "gru" else 0.0
    for x, y in zip(a, e):
        torch.testing.assert_close(x, y, atol=tol, rtol=0)


@pytest.mark.parametrize("cell", list(SIZES))
def test_cut_at_one_step(cell):
    # one step: only the initial hidden state loses its R^T dG cotangent (what
    # the reference's pointwise-only loop returns as ds0,
    # fused/flashrnn_fused_backward_cut.cu:170-178); everything else is unchanged
    leaves = rand_inputs(cell, T=1)
    a, _ = run(flashrnn_torch_fused_options, leaves, cell, gradient_recurrent_cut=True)
    e, _ = run(flashrnn_torch, leaves, cell)
    for x, y in zip(a[:5], e[:5]):
        torch.testing.assert_close(x, y, atol=0, rtol=0)
    torch.testing.assert_close(a[5][1:], e[5][1:], atol=0, rtol=0)
    if cell != "gru":  # no direct path from h_{t-1} to the new state
        assert a[5][0].abs().max() == 0 and e[5][0].abs().max() > 0


def test_elman_cut_closed_form():
    wx, R, b, s0 = rand_inputs("elman", T=6)
    (hist, last, dwx, dR, db, ds0), dh = run(flashrnn_torch_fused_options, (wx, R, b, s0), "elman",
                                             gradient_recurrent_cut=True)
    g = torch.Generator().manual_seed(7)
    dh = torch.randn(hist.shape, generator=g, dtype=hist.dtype)
    dl = torch.randn(last.shape, generator=g, dtype=last.dtype)
    dh[:, :, -1:] += dl
    h = hist[0]                                   # [B,T,N,D]
    expect = dh[0] * (1 - h * h)                  # only the caller's cotangent of h_t
    torch.testing.assert_close(dwx[:, :, 0], expect, atol=1e-12, rtol=0)
    hprev = torch.cat((s0[0].detach(), h[:, :-1]), dim=1)
    torch.testing.assert_close(dR[0], torch.einsum("btno,btnp->nop", expect, hprev), atol=1e-12, rtol=0)
    torch.testing.assert_close(db[0], expect.sum((0, 1)), atol=1e-12, rtol=0)
    torch.testing.assert_close(ds0, torch.zeros_like(ds0), atol=0, rtol=0)


def test_forward_clamp_is_straight_through():
    wx, R, b, s0 = rand_inputs("elman", T=1, scale=3.0)
    R = torch.zeros_like(R).requires_grad_()
    v = 0.5
    (hist, last, dwx, *_), _ = run(flashrnn_torch_fused_options, (wx, R, b, s0), "elman",
                                   gradient_recurrent_clipval=v)
    pre = wx.detach()[:, 0, 0] + b.detach()[0]
    torch.testing.assert_close(hist[0, :, 0], torch.tanh(pre).clamp(-v, v), atol=1e-15, rtol=0)
    assert (torch.tanh(pre).abs() > v).any()      # the clamp is active somewhere
    g = torch.Generator().manual_seed(7)
    dh = torch.randn(hist.shape, generator=g, dtype=hist.dtype)
    dl = torch.randn(last.shape, generator=g, dtype=last.dtype)
    expect = (dh[0, :, 0] + dl[0, :, 0]) * (1 - torch.tanh(pre) ** 2)
    torch.testing.assert_close(dwx[:, 0, 0], expect, atol=1e-12, rtol=0)


@pytest.mark.parametrize("cell", list(SIZES))
def test_forward_bound(cell):
    v = 0.05
    leaves = rand_inputs(cell, T=7, scale=2.0)
    (hist, last, *_), _ = run(flashrnn_torch_fused_options, leaves, cell, gradient_recurrent_clipval=v)
    assert hist[0].abs().max() <= v and last[0].abs().max() <= v
    assert hist[0].abs().max() == v  # reached


def test_gru_direct_path_is_clamped():
    """GRU at R = 0 over two steps: the cotangent of h_0 through step 1 is
    u_1 dh_1 (the direct path only), clamped; the initial state's cotangent
    u_0 (dh_0 + clamp(u_1 dh_1)) is not clamped."""
    wx, R, b, s0 = rand_inputs("gru", T=2)
    R = torch.zeros_like(R).requires_grad_()
    v = 0.01
    (hist, last, dwx, dR, db, ds0), _ = run(flashrnn_torch_fused_options, (wx, R, b, s0), "gru",
                                            gradient_recurrent_clipval=v)
    g = torch.Generator().manual_seed(7)
    dh = torch.randn(hist.shape, generator=g, dtype=hist.dtype)
    dl = torch.randn(last.shape, generator=g, dtype=last.dtype)
    u = torch.sigmoid(wx.detach()[:, :, 1] + b.detach()[2])  # [B,T,N,D]
    through = u[:, 1] * (dh[0, :, 1] + dl[0, :, 0])
    assert (through.abs() > v).any() and (u[:, 0] * (dh[0, :, 0] + through.clamp(-v, v))).abs().max() > v
    expect = u[:, 0] * (dh[0, :, 0] + through.clamp(-v, v))
    torch.testing.assert_close(ds0[0, :, 0], expect, atol=1e-15, rtol=0)


@pytest.mark.parametrize("cell", ["lstm", "slstm", "elman"])
def test_vanishing_clip_equals_cut(cell):
    leaves = rand_inputs(cell, T=6)
    v = 1e-30
    a, _ = run(flashrnn_torch_fused_options, leaves, cell, gradient_recurrent_clipval=v)
    e, _ = run(flashrnn_torch_fused_options, leaves, cell, gradient_recurrent_clipval=v, gradient_recurrent_cut=True)
    for x, y in zip(a[:5], e[:5]):
        torch.testing.assert_close(x, y, atol=1e-25, rtol=1e-12)
    # the initial state's cotangent is never clamped: only the cut removes its R^T dG part
    torch.testing.assert_close(a[5][1:], e[5][1:], atol=1e-25, rtol=1e-12)
    assert e[5][0].abs().max() == 0 and a[5][0].abs().max() > 0


# ---------------------------------------------------------------- training call
from oracle.torch_restatement import training_recurrence  # noqa: E402


@pytest.mark.parametrize("cell", list(SIZES))
@pytest.mark.parametrize("mode", ["full", "hidden", "last"])
def test_training_forward_is_flashrnn_torch(cell, mode):
    """Forward values (any gradient convention) and the output policy's selection."""
    leaves = rand_inputs(cell)
    out, fin = training_recurrence(*leaves, cell=cell, output_mode=mode)
    hist, last = flashrnn_torch(*leaves, cell=cell)
    exp = {"full": hist, "hidden": hist[0], "last": hist[0][:, -1:]}[mode]
    torch.testing.assert_close(out, exp, atol=0, rtol=0)
    torch.testing.assert_close(fin, last, atol=0, rtol=0)


@pytest.mark.parametrize("cell", ["lstm", "gru", "elman"])
def test_training_gradient_exact_without_stabilizer(cell):
    """Cells without a stabilizer or clamp: the v1 convention is the exact gradient."""
    leaves = rand_inputs(cell)
    a, _ = run(lambda *l, cell: training_recurrence(*l, cell=cell, output_mode="full"), leaves, cell)
    e, _ = run(flashrnn_torch, leaves, cell)
    for x, y in zip(a[2:], e[2:]):
        torch.testing.assert_close(x, y, atol=0, rtol=0)


def _hidden_loss_grads(fn, leaves, seed=3):
    out, fin = fn(*leaves)
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(out.shape, generator=g, dtype=out.dtype)
    wf = torch.randn(fin[0].shape, generator=g, dtype=fin.dtype)
    return torch.autograd.grad((out * w).sum() + (fin[0] * wf).sum(), leaves)


def test_slstm_v1_is_true_gradient_of_hidden_outputs():
    """grad_reference.py:8-11: h does not depend on the stabilizer m, and with n0 >= 1
    the clamp is never active (n' = f'n + i' > 1 since one of f', i' is 1); so for a
    loss on the hidden states only the v1 convention gives the exact gradient of every
    input except the initial m, whose v1 gradient is zero. The exact gradient of m0 is
    not zero here (m0 enters m_1 through log f), which the convention drops."""
    leaves = rand_inputs("slstm", T=6)  # n0 = |.| + 1 >= 1
    with torch.no_grad():
        assert (leaves[3][2] >= 1).all()
    v1 = _hidden_loss_grads(lambda *l: training_recurrence(*l, cell="slstm", output_mode="hidden"), leaves)
    ex = _hidden_loss_grads(lambda *l: training_recurrence(*l, cell="slstm", output_mode="hidden", v1_grad=False),
                            leaves)
    for x, y in zip(v1[:3], ex[:3]):
        torch.testing.assert_close(x, y, atol=1e-12, rtol=1e-10)
    torch.testing.assert_close(v1[3][:3], ex[3][:3], atol=1e-12, rtol=1e-10)
    assert v1[3][3].abs().max() == 0


def test_slstm_v1_at_the_clamp_tie():
    """From a zero state the first step's normalizer is exactly 1, the clamp's tie:
    torch.maximum gives each side half the cotangent, the straight-through clamp all
    of it. h_1 = sig(o) tanh(z) does not depend on i or n_0 otherwise, so every
    gradient agrees except the initial normalizer's, which v1 doubles; the initial m's
    is zero in both (the predicate replaces m by i at the first step)."""
    leaves = rand_inputs("slstm", T=3)
    with torch.no_grad():
        leaves[3].zero_()
    v1 = _hidden_loss_grads(lambda *l: training_recurrence(*l, cell="slstm", output_mode="hidden"), leaves)
    ex = _hidden_loss_grads(lambda *l: training_recurrence(*l, cell="slstm", output_mode="hidden", v1_grad=False),
                            leaves)
    for x, y in zip(v1[:3], ex[:3]):
        torch.testing.assert_close(x, y, atol=1e-14, rtol=1e-12)
    torch.testing.assert_close(v1[3][:2], ex[3][:2], atol=1e-14, rtol=1e-12)
    assert ex[3][2].abs().max() > 0.1
    torch.testing.assert_close(v1[3][2], 2 * ex[3][2], atol=1e-14, rtol=1e-12)
    assert v1[3][3].abs().max() == 0 and ex[3][3].abs().max() == 0

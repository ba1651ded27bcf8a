"""Pins the CPU oracle before anything is checked against it (CPU only).

Each check is chosen so that a plausible mistake in the oracle -- a dropped
term, a wrong sign, a transposed operand, a misplaced BF16 rounding -- fails
at least one of them:

* golden vectors written by the reference's own ``flashrnn_torch``
  (``tests/golden/make_golden.py``) -- BF16 policy for every cell, sLSTM;
* library known answers: ``torch.nn.LSTM/GRU/RNN`` under the gate mapping of
  ``flashrnn/flashrnn2/torch_layer.py:33-57``;
* closed forms: Elman with R=0 (``tests/flashrnn2/test_torch_backend.py:47-57``),
  the sLSTM normalizer known answer ``m = 2 - log 2``
  (``tests/flashrnn2/test_reference.py:45-63``), a single LSTM step;
* invariants: chunked == unchunked bitwise, gradcheck, BF16 policy ==
  step-by-step restatement bitwise (``test_torch_backend.py:59-124``);
* the hand-derived NumPy backward == autograd.
"""

import glob
import math
import os
from functools import partial

import numpy as np
import pytest
import torch

from oracle import numpy_explicit as ne
from oracle.torch_restatement import SIZES, flashrnn_torch, recurrence

GOLDEN = sorted(p for p in glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz"))
                if not os.path.basename(p).startswith("c1_"))
C1_FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "c1_lstm_fp32.npz")


def rand_inputs(cell, B=3, T=5, N=2, D=4, dtype=torch.float64, seed=20261005, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    gw, gt, S = SIZES[cell]
    wx = scale * torch.randn(B, T, gw, N, D, generator=g, dtype=torch.float64)
    R = scale * torch.randn(gw, N, D, D, generator=g, dtype=torch.float64) / D**0.5
    b = 0.1 * torch.randn(gt, N, D, generator=g, dtype=torch.float64)
    s0 = 0.3 * torch.randn(S, B, 1, N, D, generator=g, dtype=torch.float64)
    if cell == "slstm":
        s0[2] = s0[2].abs() + 1
    return tuple(t.to(dtype).requires_grad_() for t in (wx, R, b, s0))


# ----------------------------------------------------------------- golden vectors
@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[:-4] for p in GOLDEN])
def test_golden_vectors_bitwise(path):
    z = np.load(path, allow_pickle=False)
    cell, numerics = str(z["cell"]), str(z["numerics"])
    leaves = [torch.from_numpy(z[k]).requires_grad_() for k in ("wx", "R", "b", "s0")]
    hist, last = flashrnn_torch(*leaves, cell=cell, numerics=numerics)
    torch.testing.assert_close(hist.detach(), torch.from_numpy(z["hist"]), atol=0, rtol=0)
    torch.testing.assert_close(last.detach(), torch.from_numpy(z["last"]), atol=0, rtol=0)
    loss = (hist * torch.from_numpy(z["d_hist"])).sum() + (last * torch.from_numpy(z["d_last"])).sum()
    grads = torch.autograd.grad(loss, leaves)
    for g, k in zip(grads, ("dwx", "dR", "db", "ds0")):
        torch.testing.assert_close(g, torch.from_numpy(z[k]), atol=0, rtol=0, msg=k)


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[:-4] for p in GOLDEN])
def test_golden_vectors_explicit_backward(path):
    z = np.load(path, allow_pickle=False)
    cell, numerics = str(z["cell"]), str(z["numerics"])
    bf = numerics == "fp32_state_bf16_mma"
    args = [z[k] for k in ("wx", "R", "b", "s0")]
    hist, _ = ne.forward(*args, cell, bf)
    # The NumPy restatement sums in its own order. In the BF16 policy a sum that
    # lands next to a BF16 rounding boundary can round the other way, and the
    # flip (2^-8 relative on one operand) carries through later steps. The
    # wide cases (64-96 wide heads, 9-12 steps) have more such flips than the
    # D=8 ones, so their bound is looser. The torch restatement above matches
    # every case bit for bit.
    wide = bf and z["wx"].shape[-1] > 8
    tol = 1e-3 if wide else (2e-5 if bf else 1e-12)
    assert np.abs(hist - z["hist"]).max() / np.abs(z["hist"]).max() <= tol
    grads = ne.backward(*args, cell, z["d_hist"], z["d_last"], bf)
    for g, k in zip(grads, ("dwx", "dR", "db", "ds0")):
        e = z[k]
        assert np.abs(g - e).max() / np.abs(e).max() <= (5e-3 if wide else 1e-4 if bf else 1e-12), k


def test_golden_coverage():
    names = {os.path.basename(p)[:-4] for p in GOLDEN}
    assert {f"bf16mma_{c}" for c in SIZES} <= names
    assert {"math_slstm_zero", "math_slstm_nonzero", "math_slstm_mixed"} <= names
    assert {f"bf16mma_{c}_wide" for c in SIZES} <= names


# ------------------------------------------------------------ library known answers
def _library_module(cell, R, b, D):
    """One head mapped onto torch.nn (mapping of torch_layer.py:33-57), identity input weights."""
    kind = {"lstm": torch.nn.LSTM, "gru": torch.nn.GRU, "elman": torch.nn.RNN}[cell]
    G = R.shape[0]
    m = kind(G * D, D, batch_first=True, dtype=torch.float64)
    with torch.no_grad():
        m.weight_ih_l0.copy_(torch.eye(G * D, dtype=torch.float64)[: m.weight_ih_l0.shape[0]])
        order = [1, 2, 0] if cell == "gru" else list(range(G))
        m.weight_hh_l0.copy_(R[order].reshape(G * D, D))
        m.bias_hh_l0.zero_()
        if cell == "gru":
            # torch GRU: r,z from (x + b_ih + W_hh h + b_hh); n = tanh(x_n + b_in + r (W_hn h + b_hn))
            m.bias_ih_l0.copy_(b[[1, 2, 3]].reshape(-1))
            m.bias_hh_l0[2 * D :].copy_(b[0])
        else:
            m.bias_ih_l0.copy_(b.reshape(-1))
    return m


@pytest.mark.parametrize("cell", ["lstm", "gru", "elman"])
def test_library_known_answer(cell):
    wx, R, b, s0 = rand_inputs(cell, B=3, T=7, N=2, D=4)
    hist, last = flashrnn_torch(wx, R, b, s0, cell=cell)
    B, T, G, N, D = wx.shape
    for n in range(N):
        m = _library_module(cell, R.detach()[:, n], b.detach()[:, n], D)
        # torch.nn's GRU gate order for the input part is (r, z, n): identity map needs Wx in that order
        x = wx.detach()[:, :, :, n].reshape(B, T, G * D)
        h0 = s0.detach()[0, :, 0, n].unsqueeze(0)
        if cell == "lstm":
            out, (hT, cT) = m(x, (h0, s0.detach()[1, :, 0, n].unsqueeze(0)))
            torch.testing.assert_close(last.detach()[1, :, 0, n], cT[0], atol=1e-12, rtol=1e-12)
        else:
            out, hT = m(x, h0)
        torch.testing.assert_close(hist.detach()[0, :, :, n], out, atol=1e-12, rtol=1e-12)
        torch.testing.assert_close(last.detach()[0, :, 0, n], hT[0], atol=1e-12, rtol=1e-12)


def test_library_known_answer_gradients_lstm():
    """Gradients of the oracle equal torch.nn.LSTM's (cuDNN-free CPU path), one head."""
    wx, R, b, s0 = rand_inputs("lstm", B=2, T=6, N=1, D=3)
    hist, last = flashrnn_torch(wx, R, b, s0, cell="lstm")
    coef = torch.linspace(-1, 1, hist[0].numel(), dtype=torch.float64).reshape(hist[0].shape)
    gR, gb = torch.autograd.grad((hist[0] * coef).sum() + last.square().sum(), (R, b))
    m = _library_module("lstm", R.detach()[:, 0], b.detach()[:, 0], 3)
    x = wx.detach()[:, :, :, 0].reshape(2, 6, 12)
    out, (hT, cT) = m(x, (s0.detach()[0, :, 0, 0][None], s0.detach()[1, :, 0, 0][None]))
    loss = (out * coef[:, :, 0]).sum() + hT.square().sum() + cT.square().sum()
    loss.backward()
    torch.testing.assert_close(m.weight_hh_l0.grad.reshape(4, 3, 3), gR[:, 0], atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(m.bias_ih_l0.grad.reshape(4, 3), gb[:, 0], atol=1e-12, rtol=1e-12)


def test_config1_lstm_fp32_forward_matches_library():
    """LSTM fp32 forward, B4 T64 N1 D64, against torch.nn.LSTM."""
    g = torch.Generator().manual_seed(1)
    wx = torch.randn(4, 64, 4, 1, 64, generator=g)
    R = torch.randn(4, 1, 64, 64, generator=g) / 8.0
    b = 0.1 * torch.randn(4, 1, 64, generator=g)
    s0 = torch.randn(2, 4, 1, 1, 64, generator=g)
    hist, last = flashrnn_torch(wx, R, b, s0, cell="lstm")
    m = _library_module("lstm", R[:, 0].double(), b[:, 0].double(), 64)
    out, (hT, cT) = m(wx[:, :, :, 0].reshape(4, 64, 256).double(), (s0[0, :, 0, 0][None].double(), s0[1, :, 0, 0][None].double()))
    torch.testing.assert_close(hist[0, :, :, 0].double(), out, atol=2e-5, rtol=0)
    torch.testing.assert_close(last[1, :, 0, 0].double(), cT[0], atol=2e-5, rtol=0)


def test_config1_fixture():
    """BASELINE config 1 exactly (B4 T64 N1 D64, FP32 inputs, seed 20261001): the oracle against
    the committed torch.nn.LSTM fixture (tests/golden/make_c1.py), in FP64 to 1e-12 and in the
    FP32 mathematical policy to 1e-5 max-abs-rel."""
    z = np.load(C1_FIXTURE, allow_pickle=False)
    args = [torch.from_numpy(z[k]) for k in ("wx", "R", "b", "s0")]
    eh, el = torch.from_numpy(z["hist"]), torch.from_numpy(z["last"])
    assert eh.shape == (2, 4, 64, 1, 64) and args[0].dtype == torch.float32
    h64, l64 = flashrnn_torch(*(a.double() for a in args), cell="lstm")
    torch.testing.assert_close(h64, eh, atol=1e-12, rtol=0)
    torch.testing.assert_close(l64, el, atol=1e-12, rtol=0)
    h32, l32 = flashrnn_torch(*args, cell="lstm", numerics="mathematical")
    for a, e in ((h32, eh), (l32, el)):
        assert ((a.double() - e).abs().max() / e.abs().max()).item() <= 1e-5
    # the inputs are the ones config 1 names
    g = torch.Generator().manual_seed(20261001)
    torch.testing.assert_close(args[0], torch.randn(4, 64, 4, 1, 64, generator=g), atol=0, rtol=0)


# --------------------------------------------------------------------- closed forms
def test_elman_zero_recurrence_closed_form():
    x = torch.randn(2, 3, 1, 1, 5, dtype=torch.float64, requires_grad=True)
    R = torch.zeros(1, 1, 5, 5, dtype=torch.float64)
    b = torch.zeros(1, 1, 5, dtype=torch.float64)
    s0 = torch.randn(1, 2, 1, 1, 5, dtype=torch.float64)
    hist, last = flashrnn_torch(x, R, b, s0, cell="elman")
    torch.testing.assert_close(hist[0], x[:, :, 0].tanh(), atol=0, rtol=0)
    (g,) = torch.autograd.grad(hist.sum(), x)
    torch.testing.assert_close(g, 1 - x.detach().tanh().square())


def test_slstm_normalizer_known_answer():
    """m after one step from m=2, logsigmoid(0) = -log 2 and i = 0: m = max(0, 2 - log 2)."""
    wx = torch.zeros(1, 1, 4, 1, 2, dtype=torch.float64)
    R = torch.zeros(4, 1, 2, 2, dtype=torch.float64)
    b = torch.zeros(4, 1, 2, dtype=torch.float64)
    s = torch.zeros(4, 1, 1, 1, 2, dtype=torch.float64)
    s[2, ..., 1] = 1
    s[3] = 2
    _, last = recurrence(wx, R, b, s, "slstm")
    torch.testing.assert_close(last[3], torch.full_like(s[3], 2 - math.log(2)))


def test_slstm_zero_start_closed_form():
    """All-zero start: m1 = i, n1 = 1, c1 = tanh z, h1 = sig(o) tanh(z)."""
    wx = torch.randn(2, 1, 4, 1, 3, dtype=torch.float64)
    R = torch.randn(4, 1, 3, 3, dtype=torch.float64)
    b = torch.zeros(4, 1, 3, dtype=torch.float64)
    s = torch.zeros(4, 2, 1, 1, 3, dtype=torch.float64)
    _, last = recurrence(wx, R, b, s, "slstm")
    i, f, z, o = wx[:, 0].unbind(1)
    torch.testing.assert_close(last[3, :, 0], i, atol=0, rtol=0)
    torch.testing.assert_close(last[2, :, 0], torch.ones_like(i), atol=0, rtol=0)
    torch.testing.assert_close(last[1, :, 0], z.tanh(), atol=1e-15, rtol=0)
    torch.testing.assert_close(last[0, :, 0], o.sigmoid() * z.tanh(), atol=1e-15, rtol=0)


def test_lstm_single_step_closed_form():
    wx, R, b, s0 = (t.detach() for t in rand_inputs("lstm", T=1))
    _, last = recurrence(wx, R, b, s0, "lstm")
    h, c = s0[0, :, 0], s0[1, :, 0]
    g = wx[:, 0] + torch.stack([torch.einsum("bnp,nop->bno", h, R[k]) for k in range(4)], 1) + b
    c1 = g[:, 1].sigmoid() * c + g[:, 0].sigmoid() * g[:, 2].tanh()
    torch.testing.assert_close(last[1, :, 0], c1, atol=1e-14, rtol=0)
    torch.testing.assert_close(last[0, :, 0], g[:, 3].sigmoid() * c1.tanh(), atol=1e-14, rtol=0)


def test_maximum_tie_rule():
    """The sLSTM backward relies on torch.maximum splitting a tie's cotangent in half."""
    a = torch.tensor([1.0, 2.0, 3.0], requires_grad=True)
    b = torch.tensor([1.0, 1.0, 4.0], requires_grad=True)
    ga, gb = torch.autograd.grad(torch.maximum(a, b).sum(), (a, b))
    torch.testing.assert_close(ga, torch.tensor([0.5, 1.0, 0.0]))
    torch.testing.assert_close(gb, torch.tensor([0.5, 0.0, 1.0]))


# ----------------------------------------------------------------------- invariants
@pytest.mark.parametrize("cell", list(SIZES))
def test_chunked_equals_full_bitwise(cell):
    wx, R, b, s0 = rand_inputs(cell, T=7)
    full, last = flashrnn_torch(wx, R, b, s0, cell=cell)
    carry, parts = s0, []
    for chunk in wx.split(3, dim=1):
        h, carry = flashrnn_torch(chunk, R, b, carry, cell=cell)
        parts.append(h)
    torch.testing.assert_close(torch.cat(parts, 2), full, atol=0, rtol=0)
    torch.testing.assert_close(carry, last, atol=0, rtol=0)


@pytest.mark.parametrize("cell", list(SIZES))
def test_bf16_policy_equals_stepwise_restatement(cell):
    tensors = tuple(t.detach().float().requires_grad_() for t in rand_inputs(cell))
    wx, R, b, s0 = tensors
    actual = flashrnn_torch(*tensors, cell=cell, numerics="fp32_state_bf16_mma")
    hist, carry = [], s0
    for t in range(wx.shape[1]):
        h, carry = recurrence(wx[:, t : t + 1], R.bfloat16().float(), b, carry, cell, mma_dtype=torch.bfloat16)
        hist.append(h)
    expected = (torch.cat(hist, 2), carry)
    for a, e in zip(actual, expected):
        torch.testing.assert_close(a, e, atol=0, rtol=0)
    ga = torch.autograd.grad(actual[0].square().sum() + actual[1].sum(), tensors)
    ge = torch.autograd.grad(expected[0].square().sum() + expected[1].sum(), tensors)
    # Gradients: equal up to the order in which autograd sums three or more
    # cotangents into one state (GRU's hidden feeds three uses), i.e. FP32 rounding.
    for a, e in zip(ga, ge):
        torch.testing.assert_close(a, e, atol=1e-6, rtol=1e-6)


@pytest.mark.parametrize("cell", list(SIZES))
def test_gradcheck(cell):
    assert torch.autograd.gradcheck(
        partial(flashrnn_torch, cell=cell), rand_inputs(cell, B=1, T=2, N=1, D=2),
        eps=1e-6, atol=1e-5, rtol=1e-4, fast_mode=True,
    )


@pytest.mark.parametrize("cell", list(SIZES))
@pytest.mark.parametrize("numerics", ["mathematical", "fp32_state_bf16_mma"])
def test_explicit_backward_equals_autograd(cell, numerics):
    dtype = torch.float64 if numerics == "mathematical" else torch.float32
    wx, R, b, s0 = rand_inputs(cell, B=3, T=6, N=2, D=5, dtype=dtype, seed=7)
    hist, last = flashrnn_torch(wx, R, b, s0, cell=cell, numerics=numerics)
    g = torch.Generator().manual_seed(8)
    dh = torch.randn(hist.shape, generator=g, dtype=dtype)
    dl = torch.randn(last.shape, generator=g, dtype=dtype)
    grads = torch.autograd.grad((hist * dh).sum() + (last * dl).sum(), (wx, R, b, s0))
    npy = [t.detach().numpy() for t in (wx, R, b, s0)]
    bf = numerics != "mathematical"
    mine = ne.backward(*npy, cell, dh.numpy(), dl.numpy(), bf)
    tol = 1e-4 if bf else 1e-12
    for a, e in zip(mine, grads):
        e = e.numpy()
        assert np.abs(a - e).max() / np.abs(e).max() <= tol


def test_bf16_round_is_rne():
    x = np.array([1.0, 1.0 + 2**-8, 1.0 + 3 * 2**-8, 1.0 + 2**-9, -2.5, 3.0e38], dtype=np.float32)
    got = ne.bf16_round(x)
    want = torch.from_numpy(x).bfloat16().float().numpy()
    assert np.array_equal(got, want)


def test_rejects_invalid_contract():
    wx, R, b, s0 = (t.detach() for t in rand_inputs("lstm"))
    cases = [
        ((wx[0], R, b, s0), {}, "ranks"),
        ((wx, R.float(), b, s0), {}, "same dtype"),
        ((wx, R, b[:1], s0), {}, "bias gate"),
        ((wx, R, b, s0[:1]), {}, "initial state"),
        ((wx, R[..., :1], b, s0), {}, "recurrent weights"),
        ((wx, R, b, s0), {"cell": "unknown"}, "unsupported cell"),
        ((wx, R, b, s0), {"numerics": "x"}, "unsupported numerical"),
        ((wx, R, b, s0), {"numerics": "fp32_state_bf16_mma"}, "FP32"),
    ]
    for args, kw, msg in cases:
        with pytest.raises(ValueError, match=msg):
            flashrnn_torch(*args, **kw)


# ------------------------------------------------------- FP16 operand policy
# The FP16 kernels follow FlashRNN2's FP16 contract (FP16 inputs, FP32 compute
# and state; flashrnn/flashrnn2/state_contract.py:21-49): the policy of
# fp32_state_bf16_mma with FP16 operands. Its oracle is the restatement's
# ``recurrence`` with FP16 operand rounding; it is pinned here against the
# explicit NumPy forward and hand-derived backward, whose FP16 rounding is
# NumPy's own conversion.
def f16_policy(wx, R, b, s0, cell):
    from oracle.torch_restatement import recurrence

    return recurrence(wx, R, b, s0, cell=cell, mma_dtype=torch.float16, recurrent_mma_dtype=torch.float16)


@pytest.mark.parametrize("cell", list(SIZES))
def test_f16_policy_equals_explicit(cell):
    wx, R, b, s0 = rand_inputs(cell, B=3, T=6, N=2, D=5, dtype=torch.float32, seed=9)
    hist, last = f16_policy(wx, R, b, s0, cell)
    npy = [t.detach().numpy() for t in (wx, R, b, s0)]
    ehist, _ = ne.forward(*npy, cell, operands="f16")
    assert np.abs(hist.detach().numpy() - ehist).max() <= 2e-5
    g = torch.Generator().manual_seed(10)
    dh = torch.randn(hist.shape, generator=g)
    dl = torch.randn(last.shape, generator=g)
    grads = torch.autograd.grad((hist * dh).sum() + (last * dl).sum(), (wx, R, b, s0))
    mine = ne.backward(*npy, cell, dh.numpy(), dl.numpy(), operands="f16")
    for a, e in zip(mine, grads):
        e = e.numpy()
        assert np.abs(a - e).max() / np.abs(e).max() <= 1e-4


def test_f16_policy_rounds_operands():
    """The FP16 policy differs from the mathematical one by FP16 operand rounding only:
    with R and every hidden state exactly representable in FP16 (R = 0, so h is the
    pointwise cell of Wx + b) the two agree bitwise; with general R they differ."""
    wx, R, b, s0 = rand_inputs("elman", B=2, T=4, N=1, D=3, dtype=torch.float32, seed=11)
    with torch.no_grad():
        Rz = torch.zeros_like(R)
        s0z = torch.zeros_like(s0)
    a, _ = f16_policy(wx, Rz, b, s0z, "elman")
    e, _ = flashrnn_torch(wx, Rz, b, s0z, cell="elman")
    assert torch.equal(a, e)
    a, _ = f16_policy(wx, R, b, s0, "elman")
    e, _ = flashrnn_torch(wx, R, b, s0, cell="elman")
    assert 0 < (a - e).abs().max() < 1e-2


def test_f16_round_is_rne():
    from oracle.numpy_explicit import f16_round

    x = np.array([1.0, 1.0 + 2**-11, 1.0 + 3 * 2**-11, 1.0 + 2**-12, -2.5, 65504.0], dtype=np.float32)
    assert f16_round(x).tolist() == [1.0, 1.0, 1.0 + 4 * 2**-11, 1.0, -2.5, 65504.0]
    t = torch.from_numpy(x).to(torch.float16).float().numpy()
    assert (t == f16_round(x)).all()

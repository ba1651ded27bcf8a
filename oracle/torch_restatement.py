"""CPU restatement of the reference's ``flashrnn_torch`` oracle (test infrastructure).

Follows ``flashrnn/flashrnn2/torch_backend.py:12-67`` (validation, numerics
policy, autocast immunity) and ``flashrnn/flashrnn2/reference.py:24-114`` (the
per-step recurrence). The per-step arithmetic is kept in the same torch op
order as the reference so that forward values *and* autograd gradients agree
bit for bit; that is why the order of additions below is exactly
``(x + ry) + b`` and every step re-derives the rounded weight.

Cell formulas (``reference.py:84-113``), with ``ry[g] = sum_p R[g,n,o,p] h[p]``:

* LSTM (gates i,f,z,o): ``c' = sig(f) c + sig(i) tanh(z)``, ``h' = sig(o) tanh(c')``.
* GRU (Wx gates r,u,v; R gates cand,r,u; 4 biases):
  ``cand = ry0 + b0``, ``r = sig(x0 + ry1 + b1)``, ``u = sig(x1 + ry2 + b2)``,
  ``v = tanh(x2 + b3 + r cand)``, ``h' = u h + (1 - u) v``.
* Elman: ``h' = tanh(x + ry + b)``.
* sLSTM (states h,c,n,m): ``logf = logsigmoid(f) + m``;
  ``m' = i`` if the *global* predicate ``all(n == 0)`` holds else ``max(i, logf)``;
  ``i' = exp(i - m')``, ``f' = exp(logf - m')``, ``c' = f' c + i' tanh(z)``,
  ``n' = max(f' n + i', 1)``, ``h' = sig(o) c' / n'``.

Policy ``fp32_state_bf16_mma`` (``torch_backend.py:21-35``): FP32 inputs; the
recurrent hidden operand and R are rounded through BF16 each step, so both
cotangents are rounded through BF16 in backward.
"""

from __future__ import annotations

import torch

# (input gates G_W, bias gates G_T, states S) per cell -- reference.py:16-21
SIZES: dict[str, tuple[int, int, int]] = {
    "lstm": (4, 4, 2),
    "slstm": (4, 4, 4),
    "gru": (3, 4, 1),
    "elman": (1, 1, 1),
}


def _round_through(t: torch.Tensor, dtype: torch.dtype | None) -> torch.Tensor:
    return t if dtype is None else t.to(dtype).to(t.dtype)


def _cell_step(cell: str, x, ry, bias, state):
    """One pointwise step. ``x`` [B,G_W,N,D], ``ry`` [B,G_R,N,D], ``state`` [S,B,N,D]."""
    if cell == "elman":
        return torch.tanh(x[:, 0] + ry[:, 0] + bias[0]).unsqueeze(0)
    if cell == "gru":
        cand = ry[:, 0] + bias[0]
        reset = torch.sigmoid(x[:, 0] + ry[:, 1] + bias[1])
        update = torch.sigmoid(x[:, 1] + ry[:, 2] + bias[2])
        value = torch.tanh(x[:, 2] + bias[3] + reset * cand)
        return (update * state[0] + (1 - update) * value).unsqueeze(0)
    gi, gf, gz, go = (x + ry + bias).unbind(1)
    if cell == "lstm":
        c = torch.sigmoid(gf) * state[1] + torch.sigmoid(gi) * torch.tanh(gz)
        return torch.stack((torch.sigmoid(go) * torch.tanh(c), c))
    # sLSTM
    _, c_old, n_old, m_old = state.unbind(0)
    log_f = torch.nn.functional.logsigmoid(gf) + m_old
    all_zero = torch.all(n_old == 0)
    m = torch.where(all_zero, gi, torch.maximum(gi, log_f))
    i_act = torch.exp(gi - m)
    f_act = torch.exp(log_f - m)
    c = f_act * c_old + i_act * torch.tanh(gz)
    n = torch.maximum(f_act * n_old + i_act, torch.ones_like(n_old))
    return torch.stack((torch.sigmoid(go) * c / n, c, n, m))


def recurrence(
    wx: torch.Tensor,
    recurrent: torch.Tensor,
    bias: torch.Tensor,
    initial: torch.Tensor,
    cell: str = "lstm",
    mma_dtype: torch.dtype | None = None,
    recurrent_mma_dtype: torch.dtype | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Return (history [S,B,T,N,D], last [S,B,1,N,D]).

    ``wx`` [B,T,G_W,N,D], ``recurrent`` [G_R,N,D(out),D(in)], ``bias`` [G_T,N,D],
    ``initial`` [S,B,1,N,D]. Mirrors ``reference.py:24-114`` without the
    sequence-context extension (a persistent-kernel research feature).
    """
    batch, steps, gates, heads, width = wx.shape
    g_w, g_t, n_states = SIZES[cell]
    if steps < 1 or gates != g_w:
        raise ValueError("expected nonempty sequence and matching input gate count")
    if recurrent.shape != (gates, heads, width, width):
        raise ValueError("recurrent weights must have layout [G,N,D,P]")
    if bias.shape != (g_t, heads, width):
        raise ValueError("bias gate count does not match cell")
    if initial.shape != (n_states, batch, 1, heads, width):
        raise ValueError("initial state must have layout [S,B,1,N,D]")
    state = initial[:, :, 0]
    history = []
    for x in wx.unbind(1):
        hidden = _round_through(state[0], mma_dtype)
        weight = _round_through(recurrent, recurrent_mma_dtype)
        ry = torch.einsum("bnp,gnop->bgno", hidden, weight)
        state = _cell_step(cell, x, ry, bias, state)
        history.append(state)
    return torch.stack(history, dim=2), state.unsqueeze(2)


def flashrnn_torch(
    wx: torch.Tensor,
    recurrent: torch.Tensor,
    bias: torch.Tensor,
    initial: torch.Tensor,
    *,
    cell: str = "lstm",
    numerics: str = "mathematical",
) -> tuple[torch.Tensor, torch.Tensor]:
    """Restates ``torch_backend.py:12-67``: validation, policy, autocast off."""
    if cell not in SIZES:
        raise ValueError(f"unsupported cell: {cell}")
    if numerics not in ("mathematical", "fp32_state_bf16_mma"):
        raise ValueError(f"unsupported numerical policy: {numerics}")
    tensors = (wx, recurrent, bias, initial)
    if any(t.layout != torch.strided for t in tensors):
        raise ValueError("inputs must have strided tensor layout")
    if tuple(t.ndim for t in tensors) != (5, 4, 3, 5):
        raise ValueError("expected wx/R/b/initial ranks 5/4/3/5")
    if any(size < 1 for size in wx.shape):
        raise ValueError("batch, time, gates, heads and width must be positive")
    if wx.dtype not in (torch.float16, torch.bfloat16, torch.float32, torch.float64):
        raise ValueError("inputs must use float16, bfloat16, float32 or float64")
    if any(t.dtype != wx.dtype for t in tensors):
        raise ValueError("all inputs must have the same dtype")
    if any(t.device != wx.device for t in tensors):
        raise ValueError("all inputs must be on the same device")
    mma = None
    if numerics == "fp32_state_bf16_mma":
        if wx.dtype != torch.float32:
            raise ValueError("fp32_state_bf16_mma requires FP32 inputs")
        mma = torch.bfloat16
    with torch.autocast(wx.device.type, enabled=False):
        return recurrence(
            wx, recurrent, bias, initial, cell=cell, mma_dtype=mma, recurrent_mma_dtype=mma
        )


# ----------------------------------------------------------------------------
# Options of the reference's fused (v1) backend, restated on top of the
# flashrnn_torch cell above. flashrnn_torch itself has none of them; their
# semantics come from the v1 CUDA pointwise code and its build flags:
#
# * gradient_recurrent_clipval = v (``flashrnn/flashrnn/flashrnn.py:357-380``).
#   The build passes v as BOTH -DFLASHRNN_GRADIENT_RECURRENT_CLIPVAL and
#   -DFLASHRNN_FORWARD_CLIPVAL (``flashrnn.py:368-372`` reads
#   gradient_recurrent_clipval for the forward value too), so:
#     - forward: the new hidden state is clamped to [-v, v] after the cell
#       and the clamped value is both output and recurrent input
#       (``fused/lstm_fused_pointwise.cuh:76-80``; gru :76-80, elman :51-55,
#       slstm :100-104); the backward has no clamp mask (straight through);
#     - backward: the recurrent cotangent of h_{t-1} -- everything that
#       reaches h_{t-1} through step t (R^T dG plus the cell's direct path,
#       e.g. GRU's u * dh) -- is clamped to [-v, v] before the cotangent from
#       the caller is added (``lstm_fused_pointwise.cuh:115-124``); the
#       cotangent of the initial state is returned unclamped.
# * forward_clipval: not read by the fused build (see above), so no effect.
# * gradient_recurrent_cut (``flashrnn.py:784-787``,
#   ``fused/flashrnn_fused_backward_cut.cu:92-181``): the backward loop is
#   pointwise only -- no R^T dG reaches h_{t-1}; direct paths (c, n, GRU's
#   u * dh) and dR, db are unchanged.
#
# Parity of this restatement is pinned by tests/test_oracle.py (closed forms
# and cross-checks between the options), as no golden vectors exist for them.
class _ClampGrad(torch.autograd.Function):
    """Identity forward; backward clamps the cotangent to [-v, v]."""

    @staticmethod
    def forward(ctx, x, v):
        ctx.v = v
        return x.view_as(x)

    @staticmethod
    def backward(ctx, g):
        return g.clamp(-ctx.v, ctx.v), None


class _StraightClamp(torch.autograd.Function):
    """Forward clamps to [-v, v]; backward passes the cotangent unchanged."""

    @staticmethod
    def forward(ctx, x, v):
        return x.clamp(-v, v)

    @staticmethod
    def backward(ctx, g):
        return g, None


def recurrence_fused_options(
    wx: torch.Tensor,
    recurrent: torch.Tensor,
    bias: torch.Tensor,
    initial: torch.Tensor,
    cell: str = "lstm",
    mma_dtype: torch.dtype | None = None,
    gradient_recurrent_cut: bool = False,
    gradient_recurrent_clipval: float | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """``recurrence`` with the fused backend's cut / clip options (see above)."""
    state = initial[:, :, 0]
    history = []
    v = gradient_recurrent_clipval
    for step, x in enumerate(wx.unbind(1)):
        carried = state
        if v is not None and step > 0:
            # the recurrent cotangent of h_{t-1}: both uses inside this step. The
            # initial state's cotangent is returned unclamped (the clamp runs at
            # the start of the next pointwise step, and step 0 has none:
            # fused/flashrnn_fused_backward.cu:612-621 stores ds_inout as is)
            carried = torch.cat((_ClampGrad.apply(state[:1], float(v)), state[1:]))
        h_in = carried[0].detach() if gradient_recurrent_cut else carried[0]
        hidden = _round_through(h_in, mma_dtype)
        weight = _round_through(recurrent, mma_dtype)
        ry = torch.einsum("bnp,gnop->bgno", hidden, weight)
        state = _cell_step(cell, x, ry, bias, carried)
        if v is not None:  # forward clamp, straight-through backward
            state = torch.cat((_StraightClamp.apply(state[:1], float(v)), state[1:]))
        history.append(state)
    return torch.stack(history, dim=2), state.unsqueeze(2)


def flashrnn_torch_fused_options(
    wx, recurrent, bias, initial, *, cell="lstm", numerics="mathematical",
    gradient_recurrent_cut=False, gradient_recurrent_clipval=None,
):
    """``flashrnn_torch`` semantics plus the fused backend's cut / clip options."""
    if cell not in SIZES:
        raise ValueError(f"unsupported cell: {cell}")
    mma = torch.bfloat16 if numerics == "fp32_state_bf16_mma" else None
    with torch.autocast(wx.device.type, enabled=False):
        return recurrence_fused_options(
            wx, recurrent, bias, initial, cell=cell, mma_dtype=mma,
            gradient_recurrent_cut=gradient_recurrent_cut,
            gradient_recurrent_clipval=gradient_recurrent_clipval,
        )


# ----------------------------------------------------------------------------
# FlashRNN2's differentiable training call (``flashrnn/flashrnn2/training.py:91-124,
# 214-228``): the forward of ``recurrence`` above, the requested output policy
# taken from the state history (full [S,B,T,N,D], hidden [B,T,N,D] = history[0],
# last [B,1,N,D] = history[0][:, -1:]) plus the final carry, and gradients under
# the FlashRNN v1 convention of ``flashrnn/flashrnn2/grad_reference.py:1-60``:
# for sLSTM the stabilizer m carries no gradient (neither the new m nor the
# m_{t-1} inside log f) and the normalizer clamp max(., 1) is straight-through.
# LSTM, GRU and Elman have no stabilizer or clamp: their gradients are exact.
class _StraightMax1(torch.autograd.Function):
    """max(x, 1) in the forward, identity in the backward (grad_reference.py:20-29)."""

    @staticmethod
    def forward(ctx, x):
        return torch.maximum(x, torch.ones_like(x))

    @staticmethod
    def backward(ctx, g):
        return g


def _slstm_step_v1(x, ry, bias, state):
    gi, gf, gz, go = (x + ry + bias).unbind(1)
    _, c_old, n_old, m_old = state.unbind(0)
    log_f = torch.nn.functional.logsigmoid(gf) + m_old.detach()
    all_zero = torch.all(n_old == 0)
    m = torch.where(all_zero, gi, torch.maximum(gi, log_f)).detach()
    i_act = torch.exp(gi - m)
    f_act = torch.exp(log_f - m)
    c = f_act * c_old + i_act * torch.tanh(gz)
    n = _StraightMax1.apply(f_act * n_old + i_act)
    return torch.stack((torch.sigmoid(go) * c / n, c, n, m))


def training_recurrence(
    wx, recurrent, bias, initial, *, cell="lstm", numerics="mathematical", output_mode="hidden", v1_grad=True,
):
    """Returns (output, final [S,B,1,N,D]) of FlashRNN2's ``training.recurrence``;
    ``v1_grad=False`` gives the exact gradient of flashrnn_torch instead."""
    if output_mode not in ("full", "hidden", "last"):
        raise ValueError("output mode must be full, hidden or last")
    mma = torch.bfloat16 if numerics == "fp32_state_bf16_mma" else None
    state = initial[:, :, 0]
    history = []
    with torch.autocast(wx.device.type, enabled=False):
        for x in wx.unbind(1):
            hidden = _round_through(state[0], mma)
            weight = _round_through(recurrent, mma)
            ry = torch.einsum("bnp,gnop->bgno", hidden, weight)
            if cell == "slstm" and v1_grad:
                state = _slstm_step_v1(x, ry, bias, state)
            else:
                state = _cell_step(cell, x, ry, bias, state)
            history.append(state)
    hist = torch.stack(history, dim=2)
    out = hist if output_mode == "full" else (hist[0] if output_mode == "hidden" else hist[0][:, -1:])
    return out, state.unsqueeze(2)


# ----------------------------------------------------------------------------
# The layer around the path: input projection + recurrence. The reference
# leaves the projection to the caller (``README.md:17``); its layer contract is
# ``TorchLayer`` (``flashrnn/flashrnn2/torch_layer.py:14-80``): projection
# weight [G,N,D,I] (``torch.nn``'s weight_ih per head, ``torch_layer.py:43-45``),
# inputs [B,T,I] -> hidden history [B,T,N,D] and final states [S,B,1,N,D].
def flashrnn_layer(inputs, input_weight, recurrent, bias, initial, *, cell="lstm", numerics="mathematical",
                   wx_dtype=None):
    """Returns (hidden [B,T,N,D], final [S,B,1,N,D]). ``wx_dtype``: the dtype the
    projection's result is stored in before the recurrence reads it (None: not rounded)."""
    wx = _round_through(torch.einsum("bti,gndi->btgnd", inputs, input_weight), wx_dtype)
    hist, last = flashrnn_torch(wx, recurrent, bias, initial, cell=cell, numerics=numerics)
    return hist[0], last

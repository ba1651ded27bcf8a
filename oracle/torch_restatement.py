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

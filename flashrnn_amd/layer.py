"""Input projection + fused recurrence: the layer around the recurrent path.

The reference's recurrence takes the projected inputs ``Wx = W x`` and leaves
the projection to the caller (``README.md:17``: "Typically the inputs are
modified with a linear layer which is omitted here"). Its layer-level contract
is ``TorchLayer`` (``flashrnn/flashrnn2/torch_layer.py:14-80``): projection
weight ``[G,N,D,I]``, recurrent weight ``[G,N,D,D]``, bias ``[G_T,N,D]``; inputs
``[B,T,I]`` and an initial state ``[S,B,1,N,D]`` give the hidden history
``[B,T,N,D]`` and the final states ``[S,B,1,N,D]``. ``FlashRNNLayer`` keeps
that contract on this library's kernels:

* the projection is one library GEMM (hipBLASLt through ``torch.matmul``) of
  ``[B*T, I] x [I, G*N*D]``, whose row-major result is already the kernels'
  ``Wx [B,T,G,N,D]`` layout: nothing is permuted;
* the recurrence runs with the hidden-state output policy (``FRNN_OUT_HIDDEN``:
  one state written per step) and returns the FP32 carry as the final states;
* gradients flow to the inputs, the three weights and the initial state; the
  recurrence's follow ``flashrnn_torch`` exactly (also for sLSTM), as
  ``flashrnn()``'s do;
* ``chunks`` (a pipeline of the projection of time chunk c+1 on a second
  stream with the recurrence of chunk c through a step window) is switched
  off: its first large-batch run on the MI355X (B256 T1024 N8 D128, I1024,
  four chunks) ended in a GPU memory fault whose cause is not found yet, so
  that code is taken out and a call with more than one chunk raises
  ``NotImplementedError``.

Differences from ``TorchLayer``, on purpose: every cell (TorchLayer maps LSTM,
GRU and Elman onto ``torch.nn`` modules, so it has no sLSTM); one call for all
heads instead of a module per head; the compute dtype is a choice (BF16 or
FP16 operands with FP32 state, or FP32), not the parameters' dtype.
"""

from __future__ import annotations

import torch
from torch import nn

from .flashrnn import CELL_SIZES, DTYPES
from .prepared import KernelConfig, default_config
from .training import _recurrence


def _check(inputs, input_weight, recurrent, bias, initial, cell):
    if cell not in CELL_SIZES:
        raise ValueError(f"unknown cell {cell!r}")
    gr, gw, gt, S = CELL_SIZES[cell]
    if input_weight.ndim != 4 or input_weight.shape[0] != gw:
        raise ValueError(f"input weight must have layout [G,N,D,I] with G = {gw} for {cell}")
    _, N, D, I = input_weight.shape
    if recurrent.shape != (gr, N, D, D) or bias.shape != (gt, N, D):
        raise ValueError("invalid recurrent-weight or bias shape")
    if inputs.ndim != 3 or inputs.shape[2] != I or min(inputs.shape) < 1:
        raise ValueError(f"inputs must have layout [B,T,I] with I = {I}")
    B = inputs.shape[0]
    if initial is not None and initial.shape != (S, B, 1, N, D):
        raise ValueError("invalid initial-state shape")
    tensors = (inputs, input_weight, recurrent, bias) + (() if initial is None else (initial,))
    if not inputs.is_cuda or any(t.device != inputs.device for t in tensors):
        raise ValueError("inputs and weights must be on one GPU device")


def project(inputs, input_weight):
    """``Wx[B,T,G,N,D] = sum_i x[B,T,i] W[G,N,D,i]``: one GEMM in the operands' dtype."""
    G, N, D, I = input_weight.shape
    B, T, _ = inputs.shape
    return torch.matmul(inputs, input_weight.reshape(G * N * D, I).t()).view(B, T, G, N, D)


def flashrnn_projected(inputs, input_weight, recurrent, bias, initial=None, cell="lstm", *, dtype="bfloat16",
                       config=None, chunks=None):
    """Projection + recurrence. Returns ``(hidden [B,T,N,D], final [S,B,1,N,D])``;
    ``final`` is the FP32 carry, ``hidden`` has the compute dtype."""
    _check(inputs, input_weight, recurrent, bias, initial, cell)
    if dtype not in DTYPES:
        raise ValueError(f"dtype {dtype!r} not supported; use one of {tuple(DTYPES)}")
    cdt = DTYPES[dtype]
    S = CELL_SIZES[cell][3]
    B, T, _ = inputs.shape
    _, N, D, _ = input_weight.shape
    if initial is None:
        initial = torch.zeros((S, B, 1, N, D), dtype=torch.float32, device=inputs.device)
    x, W, R, b = (t.to(cdt) for t in (inputs, input_weight, recurrent, bias))
    config = config or default_config(D)
    if not isinstance(config, KernelConfig):
        raise ValueError("config must be a flashrnn_amd.prepared.KernelConfig")
    grad = torch.is_grad_enabled() and any(t.requires_grad for t in (inputs, input_weight, recurrent, bias, initial))
    lengths = (T,) if chunks is None else tuple(chunks)
    if not lengths or any(type(n) is not int or n < 1 for n in lengths) or sum(lengths) != T:
        raise ValueError("chunk lengths must be positive integers totaling T")
    if len(lengths) > 1:
        raise NotImplementedError("the chunked projection pipeline is switched off (an unresolved GPU memory "
                                  "fault at B256 T1024); call without chunks")
    # one projection, then the differentiable recurrence (exact gradients)
    return _recurrence(project(x, W), R, b, initial, cell, "hidden", None, config, v1=False)


class FlashRNNLayer(nn.Module):
    """``TorchLayer``'s contract (``torch_layer.py:14-80``) on the fused kernels: the
    parameters are copied once at construction; ``forward(inputs, initial)`` returns the
    hidden history ``[B,T,N,D]`` and the final states ``[S,B,1,N,D]``."""

    def __init__(self, input_weight, recurrent, bias, cell, *, dtype="bfloat16", config=None):
        super().__init__()
        if cell not in CELL_SIZES:
            raise ValueError(f"unknown cell {cell!r}")
        gr, gw, gt, _ = CELL_SIZES[cell]
        if input_weight.ndim != 4 or input_weight.shape[0] != gw:
            raise ValueError("invalid gate or input-weight shape")
        _, N, D, _ = input_weight.shape
        if recurrent.shape != (gr, N, D, D):
            raise ValueError("invalid gate or recurrent-weight shape")
        if bias.shape != (gt, N, D):
            raise ValueError("invalid bias shape")
        if dtype not in DTYPES:
            raise ValueError(f"dtype {dtype!r} not supported; use one of {tuple(DTYPES)}")
        self.cell, self.dtype, self.config = cell, dtype, config
        self.input_weight = nn.Parameter(input_weight.detach().clone())
        self.recurrent = nn.Parameter(recurrent.detach().clone())
        self.bias = nn.Parameter(bias.detach().clone())

    def forward(self, inputs, initial=None, *, chunks=None):
        return flashrnn_projected(inputs, self.input_weight, self.recurrent, self.bias, initial, self.cell,
                                  dtype=self.dtype, config=self.config, chunks=chunks)

"""Input projection + fused recurrence: the layer around the recurrent path.

The reference's recurrence takes the projected inputs ``Wx = W x`` and leaves
the projection to the caller (``README.md:17``: "Typically the inputs are
modified with a linear layer which is omitted here"). Its layer-level contract
is ``TorchLayer`` (``flashrnn/flashrnn2/torch_layer.py:14-80``): projection
weight ``[G,N,D,I]``, recurrent weight ``[G,N,D,D]``, bias ``[G_T,N,D]``; inputs
``[B,T,I]`` and an initial state ``[S,B,1,N,D]`` give the hidden history
``[B,T,N,D]`` and the final states ``[S,B,1,N,D]``. ``FlashRNNLayer`` keeps
that contract on this library's kernels:

* the projection ``Wx[B,T,G,N,D] = x W^T`` runs in the recurrence's own launch
  (``frnn_fwd_projected``): hand-written MFMA workers on the CUs the
  recurrence leaves free compute Wx in time order, and the recurrence's I/O
  waves read each step's rows as soon as they are complete, so the projection
  costs the forward almost nothing where the recurrence leaves whole XCDs
  free. 16-bit compute dtypes, head widths that are multiples of 32 and input
  sizes that are multiples of 8 can take this path; by default calls without
  a backward and with fewer than eight head x batch-slab groups do (see
  ``flashrnn_projected``); otherwise the projection is one library GEMM (``torch.matmul``) of
  ``[B*T, I] x [I, G*N*D]``, whose row-major result is already the kernels'
  Wx layout;
* the recurrence runs with the hidden-state output policy (``FRNN_OUT_HIDDEN``:
  one state written per step) and returns the FP32 carry as the final states;
* gradients flow to the inputs, the three weights and the initial state; the
  recurrence's follow ``flashrnn_torch`` exactly (also for sLSTM), as
  ``flashrnn()``'s do; ``dx = dWx W`` and ``dW = dWx^T x`` are library GEMMs
  after the backward recurrence.

Differences from ``TorchLayer``, on purpose: every cell (TorchLayer maps LSTM,
GRU and Elman onto ``torch.nn`` modules, so it has no sLSTM); one call for all
heads instead of a module per head; the compute dtype is a choice (BF16 or
FP16 operands with FP32 state, or FP32), not the parameters' dtype.
"""

from __future__ import annotations

import torch
from torch import nn

from . import _lib
from .flashrnn import _IO, _MMA_OF, CELL_SIZES, DTYPES, _after_call, _drain_pending, _workspace
from .prepared import KernelConfig, default_config
from .training import _backward, _flags, _recurrence


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
    """``Wx[B,T,G,N,D] = sum_i x[B,T,i] W[G,N,D,i]``: one library GEMM in the operands' dtype."""
    G, N, D, I = input_weight.shape
    B, T, _ = inputs.shape
    return torch.matmul(inputs, input_weight.reshape(G * N * D, I).t()).view(B, T, G, N, D)


class _ProjectedRecurrence(torch.autograd.Function):
    """Projection + recurrence through ``frnn_fwd_projected`` (one launch where the
    recurrence leaves CUs free); backward: ``frnn_bwd``, then dx and dW as GEMMs."""

    @staticmethod
    def forward(ctx, x, W, recurrent, bias, initial, cell, config, grad):
        _drain_pending()
        lib = _lib.load()
        B, T, I = x.shape
        G, N, D, _ = W.shape
        S = CELL_SIZES[cell][3]
        dev = x.device
        training = grad  # a backward can follow (grad mode on at the call, an input requires grad)
        flags = _flags("hidden", False, cell, config, training, v1=False)
        d = _lib.FrnnDesc(_lib.CELLS[cell], B, T, N, D, _IO[x.dtype], _lib.FRNN_F32, _MMA_OF[x.dtype], flags,
                          0.0, 0, 0)
        s0 = initial[:, :, 0].to(torch.float32).contiguous()
        wx = torch.empty((B, T, G, N, D), dtype=x.dtype, device=dev)
        hist = torch.empty((B, T, N, D), dtype=x.dtype, device=dev)
        carry = torch.empty((S, B, N, D), dtype=torch.float32, device=dev)
        ws = _workspace(lib.frnn_workspace_bytes(d, 3), dev)
        save = torch.empty(lib.frnn_workspace_bytes(d, 2), dtype=torch.uint8, device=dev) if training else None
        stream = torch.cuda.current_stream(dev).cuda_stream
        rc = lib.frnn_fwd_projected(d, I, x.data_ptr(), W.data_ptr(), wx.data_ptr(), recurrent.data_ptr(),
                                    bias.data_ptr(), s0.data_ptr(), hist.data_ptr(), carry.data_ptr(),
                                    save.data_ptr() if save is not None else None, ws.data_ptr(), ws.numel(), stream)
        _lib.check(rc, "frnn_fwd_projected")
        _after_call(ws)
        if training:
            ctx.save_for_backward(x, W, recurrent, s0, hist, save)
            ctx.meta = (d, wx.shape, bias.shape, initial.dtype)
        return hist, carry.unsqueeze(2)

    @staticmethod
    def backward(ctx, d_out, d_final):
        x, W, recurrent, s0, hist, save = ctx.saved_tensors
        d, wshape, bshape, init_dtype = ctx.meta
        dwx, dR, db, ds0 = _backward(d, recurrent, s0, hist, save, d_out, d_final, wshape, x.dtype, bshape, "hidden")
        B, T, I = x.shape
        G, N, D, _ = W.shape
        dg = dwx.view(B * T, G * N * D)
        dx = (dg @ W.view(G * N * D, I)).view(B, T, I)
        dW = (dg.t() @ x.reshape(B * T, I)).view(G, N, D, I)
        return dx, dW, dR, db, ds0.unsqueeze(2).to(init_dtype), None, None, None


def flashrnn_projected(inputs, input_weight, recurrent, bias, initial=None, cell="lstm", *, dtype="bfloat16",
                       config=None, overlap=None):
    """Projection + recurrence. Returns ``(hidden [B,T,N,D], final [S,B,1,N,D])``;
    ``final`` is the FP32 carry, ``hidden`` has the compute dtype. ``overlap``: True runs
    the projection in the recurrence's launch wherever the kernels allow it, False as a
    library GEMM before the recurrence, None (default) in the launch where that was
    measured faster: calls without a backward (no gradient recorded) and fewer than
    eight head x batch-slab groups."""
    _check(inputs, input_weight, recurrent, bias, initial, cell)
    if dtype not in DTYPES:
        raise ValueError(f"dtype {dtype!r} not supported; use one of {tuple(DTYPES)}")
    cdt = DTYPES[dtype]
    S = CELL_SIZES[cell][3]
    B, T, I = inputs.shape
    _, N, D, _ = input_weight.shape
    if initial is None:
        initial = torch.zeros((S, B, 1, N, D), dtype=torch.float32, device=inputs.device)
    x, W, R, b = (t.to(cdt) for t in (inputs, input_weight, recurrent, bias))
    config = config or default_config(D)
    if not isinstance(config, KernelConfig):
        raise ValueError("config must be a flashrnn_amd.prepared.KernelConfig")
    grad = torch.is_grad_enabled() and any(t.requires_grad for t in (x, W, R, b, initial))
    # The projection's workers pay where the recurrence leaves whole XCDs free (fewer than
    # eight head x batch-slab groups) and the forward saves nothing for a backward: measured
    # at B16 T1024 I768, NH*DH = 768, 8% faster than the library GEMM at NH 6 and 7% slower
    # at NH 12 (every XCD holds groups); at B8 T1024 N3 D256 I768 6% faster without a
    # backward, 1.5% slower with one.
    if overlap is None:
        overlap = not grad and N * ((B + 15) // 16) < 8
    if overlap and cdt != torch.float32 and D % 32 == 0 and D <= 1024 and I % 8 == 0:
        return _ProjectedRecurrence.apply(x.contiguous(), W.contiguous(), R.contiguous(), b.contiguous(), initial,
                                          cell, config, grad)
    # one library projection, then the differentiable recurrence (exact gradients)
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

    def forward(self, inputs, initial=None, *, overlap=None):
        return flashrnn_projected(inputs, self.input_weight, self.recurrent, self.bias, initial, self.cell,
                                  dtype=self.dtype, config=self.config, overlap=overlap)

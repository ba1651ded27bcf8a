"""FlashRNN2's differentiable whole-call recurrence with an output policy.

Mirrors ``recurrence`` of ``flashrnn/flashrnn2/training.py:214-228`` (and its
autograd function ``_Recurrence``, ``training.py:91-210``) on this library's
kernels: ``recurrence(wx, recurrent, bias, initial, cell, output_mode=...,
snapshot_dtype=...)`` returns ``(output, final)`` where

* ``output`` is the state history ``[S,B,T,N,D]`` (``"full"``), the hidden
  state history ``[B,T,N,D]`` (``"hidden"``, the default) or the last hidden
  state ``[B,1,N,D]`` (``"last"``), in ``snapshot_dtype`` (input dtype or FP32);
* ``final`` is the FP32 compute carry ``[S,B,1,N,D]``;

and gradients flow to all four inputs, returned in their dtypes. As in the
reference, gradients follow the FlashRNN v1 convention
(``flashrnn/flashrnn2/grad_reference.py:1-12``): for sLSTM the stabilizer m
carries no gradient and the normalizer clamp is straight-through
(``FRNN_SLSTM_V1GRAD``); the other cells' gradients are exact.

The forward writes only what the backward needs: the hidden history alone for
the ``hidden`` and ``last`` policies (``FRNN_OUT_HIDDEN``; the backward's dR
GEMM reads nothing else), in FP32 when ``snapshot_dtype`` is FP32. ``last``
returns the final step of that history, and its cotangent joins the carry's.

Differences from the reference, on purpose: every cell of the fused path is
accepted (the reference trains LSTM and sLSTM only); inputs are BF16 or FP16
(16-bit recurrent-product operands, FP32 accumulation and state) or FP32 (FP32
product); ``config`` is :class:`flashrnn_amd.prepared.KernelConfig`;
``backward_options`` (the reference's Triton/CUDA backward tuning knobs) must be
empty: this backward has one kernel. A ``sequence_context`` past the first step
is refused, as in the reference (``training.py:223-224``).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib
from .flashrnn import _IO, _MMA_OF, CELL_SIZES, _after_call, _drain_pending, _state, _workspace
from .prepared import KernelConfig, default_config


def _flags(output_mode, snap32, cell, config, training, v1=True):
    exchange = config.exchange or ("shared" if _state["xcd_shared"] else "xcd")
    flags = _lib.FRNN_TRAINING if training else 0
    flags |= _lib.FRNN_OUT_HIDDEN if output_mode != "full" else 0
    flags |= _lib.FRNN_SNAPSHOT_F32 if snap32 else 0
    flags |= _lib.FRNN_SLSTM_V1GRAD if cell == "slstm" and v1 else 0
    flags |= _lib.FRNN_XCD_SHARED if exchange == "shared" else 0
    flags |= _lib.FRNN_TEST_UNREADY if _state["test_unready"] else 0
    return flags


class _Recurrence(torch.autograd.Function):
    @staticmethod
    def forward(ctx, wx, recurrent, bias, initial, cell, output_mode, snapshot_dtype, config, v1, grad):
        _drain_pending()
        lib = _lib.load()
        B, T, _, N, D = wx.shape
        S = CELL_SIZES[cell][3]
        dev = wx.device
        snap = wx.dtype if snapshot_dtype is None else snapshot_dtype
        training = grad  # a backward can follow (grad mode on at the call, an input requires grad)
        flags = _flags(output_mode, snap == torch.float32 and snap != wx.dtype, cell, config, training, v1)
        mma = _MMA_OF[wx.dtype]
        d = _lib.FrnnDesc(_lib.CELLS[cell], B, T, N, D, _IO[wx.dtype], _lib.FRNN_F32, mma, flags, 0.0, 0, 0)
        s0 = initial[:, :, 0].to(torch.float32).contiguous()  # exact; the carry is FP32
        hist = torch.empty((S, B, T, N, D) if output_mode == "full" else (B, T, N, D), dtype=snap, device=dev)
        carry = torch.empty((S, B, N, D), dtype=torch.float32, device=dev)
        ws = _workspace(lib.frnn_workspace_bytes(d, 0), dev)
        save = torch.empty(lib.frnn_workspace_bytes(d, 2), dtype=torch.uint8, device=dev) if training else None
        stream = torch.cuda.current_stream(dev).cuda_stream
        rc = lib.frnn_fwd(d, wx.data_ptr(), recurrent.data_ptr(), bias.data_ptr(), s0.data_ptr(), hist.data_ptr(),
                          carry.data_ptr(), save.data_ptr() if save is not None else None, ws.data_ptr(), ws.numel(),
                          stream)
        _lib.check(rc, "frnn_fwd")
        _after_call(ws)
        if training:
            ctx.save_for_backward(recurrent, s0, hist, save)
            ctx.meta = (d, wx.shape, wx.dtype, bias.shape, initial.dtype, output_mode)
        out = hist[:, -1:].clone() if output_mode == "last" else hist
        return out, carry.unsqueeze(2)

    @staticmethod
    def backward(ctx, d_out, d_final):
        recurrent, s0, hist, save = ctx.saved_tensors
        d, wshape, io, bshape, init_dtype, output_mode = ctx.meta
        dwx, dR, db, ds0 = _backward(d, recurrent, s0, hist, save, d_out, d_final, wshape, io, bshape, output_mode)
        return dwx, dR, db, ds0.unsqueeze(2).to(init_dtype), None, None, None, None, None, None


def _backward(d, recurrent, s0, hist, save, d_out, d_final, wshape, io, bshape, output_mode):
    """frnn_bwd of a training forward: (dWx, dR, db, ds0 [S,B,N,D] FP32) from the
    cotangents of its output (``d_out``, per ``output_mode``) and of its FP32 carry."""
    _drain_pending()
    lib = _lib.load()
    dev = recurrent.device
    d_carry = d_final[:, :, 0].float().contiguous() if d_final is not None else None
    d_states = None
    if d_out is not None:
        if output_mode == "last":  # the last hidden state is the carry's h (rounded): its cotangent joins d_carry
            extra = d_out[:, 0].float()
            if d_carry is None:
                d_carry = torch.zeros(s0.shape, dtype=torch.float32, device=dev)
            d_carry[0] += extra
        else:
            d_states = d_out.to(hist.dtype).contiguous()
    dwx = torch.empty(wshape, dtype=io, device=dev)
    dR = torch.empty(recurrent.shape, dtype=io, device=dev)
    db = torch.empty(bshape, dtype=io, device=dev)
    ds0 = torch.empty(s0.shape, dtype=torch.float32, device=dev)
    ws = _workspace(lib.frnn_workspace_bytes(d, 1), dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = lib.frnn_bwd(d, recurrent.data_ptr(), s0.data_ptr(), hist.data_ptr(), save.data_ptr(),
                      d_states.data_ptr() if d_states is not None else None,
                      d_carry.data_ptr() if d_carry is not None else None,
                      dwx.data_ptr(), dR.data_ptr(), db.data_ptr(), ds0.data_ptr(), ws.data_ptr(), ws.numel(),
                      stream)
    _lib.check(rc, "frnn_bwd")
    _after_call(ws)
    return dwx, dR, db, ds0


def recurrence(wx, recurrent, bias, initial, cell="lstm", *, output_mode="hidden", snapshot_dtype=None, config=None,
               sequence_context=None, backward_options=None):
    """Differentiable whole-call recurrence. Returns (output, FP32 final carry)."""
    if sequence_context is not None and getattr(sequence_context, "step_offset", 0) > 0:
        raise ValueError("a continuation chunk cannot be differentiated; run the whole logical call")
    if backward_options:
        raise ValueError("backward_options are tuning knobs of the reference's CUDA/Triton backwards; "
                         "this backward has none")
    return _recurrence(wx, recurrent, bias, initial, cell, output_mode, snapshot_dtype, config, v1=True)


def _recurrence(wx, recurrent, bias, initial, cell, output_mode, snapshot_dtype, config, v1):
    """``recurrence`` with the sLSTM gradient convention as a choice: v1 (FlashRNN2's
    training) or exact (flashrnn_torch's, as ``flashrnn()`` uses)."""
    if cell not in CELL_SIZES:
        raise ValueError(f"unknown cell {cell!r}")
    if output_mode not in ("full", "hidden", "last"):
        raise ValueError("output mode must be full, hidden or last")
    if snapshot_dtype not in (None, wx.dtype, torch.float32):
        raise ValueError("snapshot dtype must be input dtype or FP32")
    gr, gw, gt, S = CELL_SIZES[cell]
    if wx.ndim != 5:
        raise ValueError(f"expected Wx [B,T,{gw},H,D]")
    B, T, G, N, D = wx.shape
    if G != gw or min(B, T, N, D) < 1:
        raise ValueError(f"expected nonempty B/T/H/D and {gw} gates for {cell}")
    if recurrent.shape != (gr, N, D, D) or bias.shape != (gt, N, D):
        raise ValueError("invalid recurrent-weight or bias shape")
    if initial.shape != (S, B, 1, N, D):
        raise ValueError("invalid initial-state shape")
    if wx.dtype not in _IO:
        raise ValueError("inputs must be bfloat16, float16 or float32")
    if recurrent.dtype != wx.dtype or bias.dtype != wx.dtype or initial.dtype not in (wx.dtype, torch.float32):
        raise ValueError("input dtype does not match generic computation contract")
    if not wx.is_cuda or any(t.device != wx.device for t in (recurrent, bias, initial)):
        raise ValueError("inputs must be on one GPU device")
    config = config or default_config(D)
    if not isinstance(config, KernelConfig):
        raise ValueError("config must be a flashrnn_amd.prepared.KernelConfig")
    # width: the kernels tile hidden units by 32; inert padding units (zero
    # weights, inputs and states) never reach a real unit
    Dp = (D + 31) // 32 * 32
    if Dp > 1024:
        raise ValueError(f"head width {D} exceeds the supported maximum 1024")
    args = [wx, recurrent, bias, initial]
    if Dp != D:
        pad = Dp - D
        args = [F.pad(wx, (0, pad)), F.pad(recurrent, (0, pad, 0, pad)), F.pad(bias, (0, pad)),
                F.pad(initial, (0, pad))]
    grad = torch.is_grad_enabled() and any(t.requires_grad for t in args)
    out, final = _Recurrence.apply(*(t.contiguous() for t in args), cell, output_mode, snapshot_dtype, config, v1,
                                   grad)
    if Dp != D:
        out, final = out[..., :D], final[..., :D]
    return out, final

"""Public entry point: ``flashrnn(Wx, R, b, states, function, config, backend, dtype)``.

Drop-in for the reference's ``flashrnn()`` (``flashrnn/flashrnn/flashrnn.py:1117-1138``)
on its fused backend: same signature, same public layouts, same return value
``(states [S,B,T,N,D], last [S,B,1,N,D])``, gradients to all four inputs.
The work runs in ``libfrnn.so`` (hand-written gfx950 HIP kernels) through the
C ABI of ``include/frnn.h``; PyTorch provides device memory and the stream.

Shapes (``flashrnn/flashrnn/flashrnn.py:45-70``): ``Wx [B,T,G_W,N,D]``, ``R [G_R,N,D,D]`` (output
index before input index), ``b [G_T,N,D]``, ``states [S,B,1,N,D]``; per cell
``(G_R, G_W, G_T, S)`` = lstm (4,4,4,2), slstm (4,4,4,4), gru (3,3,4,1),
elman (1,1,1,1).

Numerics. ``dtype="bfloat16"`` (the default, as in the reference) runs the
recurrent product with BF16 operands and FP32 accumulation and keeps every
state and the pointwise cell in FP32: the reference's
``numerics="fp32_state_bf16_mma"`` policy (``flashrnn2/torch_backend.py:21-35``).
``dtype="float16"`` does the same with FP16 operands (FlashRNN2's FP16
contract: FP16 inputs, FP32 compute and state). ``dtype="float32"`` runs the
product in FP32 (the mathematical policy).
Inputs may be BF16, FP16 or FP32 in either mode; the state history uses the
dtype of ``Wx``. When ``Wx``, ``R`` and ``b`` differ in dtype, all three are
promoted to FP32 for the call (``io_dtype``), so an FP32 ``R`` or ``b`` is
never rounded to ``Wx``'s 16-bit type before the policy rounds the operands.

``last`` is the full-precision carry: it has the dtype of the ``states``
argument (FP32 carries in give FP32 carries out), so chunked calls continue
exactly where the unchunked call would be (``docs/flashrnn2/persistent-continuation.md``).
"""

from __future__ import annotations

import collections
import os
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn.functional as F

from . import _lib

# (G_R, G_W, G_T, S); rnn_function_registry, flashrnn/flashrnn/flashrnn.py:45-70
CELL_SIZES = {"lstm": (4, 4, 4, 2), "slstm": (4, 4, 4, 4), "gru": (3, 3, 4, 1), "elman": (1, 1, 1, 1)}
FUSED_BACKENDS = ("cuda_fused", "fused", "hip_fused")
DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}
_IO = {torch.float32: _lib.FRNN_F32, torch.bfloat16: _lib.FRNN_BF16, torch.float16: _lib.FRNN_F16}
# recurrent-product operand type of a config dtype (or of an input dtype)
_MMA = {"bfloat16": _lib.FRNN_MMA_BF16, "float16": _lib.FRNN_MMA_F16, "float32": _lib.FRNN_MMA_F32}
_MMA_OF = {torch.bfloat16: _lib.FRNN_MMA_BF16, torch.float16: _lib.FRNN_MMA_F16, torch.float32: _lib.FRNN_MMA_F32}


@dataclass
class FlashRNNConfig:
    """The subset of the reference's ``FlashRNNConfig`` (``flashrnn/flashrnn/flashrnn.py:121-380``)
    that applies to the fused path.

    ``gradient_recurrent_cut`` and ``gradient_recurrent_clipval`` behave as on
    the reference's fused backend (``flashrnn.py:357-380, 784-787``): the cut
    passes no ``R^T dG`` cotangent to ``h_{t-1}``; a clip value ``v`` clamps
    every new hidden state to ``[-v, v]`` (straight-through in backward: the
    fused build passes ``gradient_recurrent_clipval`` as its forward clip
    value, ``flashrnn.py:368-372``) and clamps the recurrent cotangent of
    ``h_{t-1}`` to the same interval before the caller's cotangent is added.
    ``forward_clipval`` is accepted and, as on the reference's fused backend,
    has no effect.

    The caller-side layouts behave as in the reference (``flashrnn.py:162-170``,
    permuted with ``permute_to`` at ``:97-108, 320-331``): ``input_shape``
    (``"BTGHD"`` or ``"TBGHD"``), ``output_shape`` (any order of S, B, T, H, D;
    default ``"SBTHD"``; the initial ``states`` argument and ``last`` use it
    too, with T = 1), ``recurrent_shape`` (any order of G, H, D, P; default
    ``"GHDP"``) and ``bias_shape`` (any order of G, H, D; default ``"GHD"``).
    ``initial_val`` (a float or one per state) fills the initial state when
    ``states`` is ``None`` (``_zero_state``, ``:930-957``). The other fields
    of the reference's config are accepted for compatibility. ``constants``
    must be empty (no cell here has any); ``dtype_acc`` must be FP32, the
    accumulation type of every kernel. ``dtype_w`` / ``dtype_r`` /
    ``dtype_b`` and the rest are informational: the tensors' own dtypes
    decide (``io_dtype``)."""

    backend: str = "cuda_fused"
    function: str = "lstm"
    dtype: str = "bfloat16"
    gradient_recurrent_cut: bool = False
    gradient_recurrent_clipval: Optional[float] = None
    forward_clipval: Optional[float] = None
    constants: Optional[dict] = None
    simple_agg: bool = True
    hidden_dim: int = -1
    num_heads: int = -1
    head_dim: int = -1
    batch_size: int = -1
    input_shape: str = "BTGHD"
    output_shape: str = "SBTHD"
    recurrent_shape: str = "GHDP"
    bias_shape: str = "GHD"
    dtype_acc: Optional[str] = "float32"
    dtype_b: Optional[str] = None
    dtype_r: Optional[str] = None
    dtype_w: Optional[str] = None
    dtype_g: Optional[str] = None
    dtype_s: Optional[str] = None
    dtype_a: Optional[str] = None
    enable_automatic_mixed_precision: bool = True
    trainable_r: object = True
    trainable_b: object = True
    initial_val: object = 0.0

    def __post_init__(self):
        if self.function not in CELL_SIZES:
            raise ValueError(f"RNN function {self.function} not in registry")
        if self.backend not in FUSED_BACKENDS:
            raise ValueError(
                f"backend {self.backend!r} is not provided by flashrnn_amd; "
                f"use one of {FUSED_BACKENDS} (the HIP fused recurrence)"
            )
        if self.dtype not in DTYPES:
            raise ValueError(f"dtype {self.dtype!r} not supported; use one of {tuple(DTYPES)}")
        v = self.gradient_recurrent_clipval
        if v is not None and not (float(v) >= 0.0 and float(v) < float("inf")):
            raise ValueError(f"gradient_recurrent_clipval must be finite and >= 0, got {v}")
        (self.num_gates_r, self.num_gates_w, self.num_gates_t, self.num_states) = CELL_SIZES[self.function]
        if self.input_shape not in ("BTGHD", "TBGHD"):
            raise ValueError(f"input_shape must be 'BTGHD' or 'TBGHD', got {self.input_shape!r}")
        for name, letters in (("output_shape", "SBTHD"), ("recurrent_shape", "GHDP"), ("bias_shape", "GHD")):
            v = getattr(self, name)
            if not isinstance(v, str) or sorted(v) != sorted(letters):
                raise ValueError(f"{name} must order the letters {letters}, got {v!r}")
        if self.constants:
            raise ValueError(f"cell {self.function} has no constants, got {self.constants!r}")
        self.constants = {}
        self.simple_agg = self.function != "gru"  # the registry's value (flashrnn.py:45-70)
        if self.dtype_acc not in (None, "float32"):
            raise ValueError(f"dtype_acc must be float32 (every kernel accumulates in FP32), got {self.dtype_acc!r}")
        iv = self.initial_val
        if not isinstance(iv, (int, float)) and len(iv) != self.num_states:
            raise ValueError(f"initial_val needs one value per state ({self.num_states}), got {iv!r}")


# ----------------------------------------------------------------- status handling
_state = {"xcd_shared": os.environ.get("FRNN_XCD_SHARED", "0") == "1",
          "strict": os.environ.get("FRNN_SYNC_CHECK", "0") == "1",
          "test_unready": False}  # failure-handling tests only (FRNN_TEST_UNREADY)
_pending: collections.deque = collections.deque()


def set_strict(flag: bool) -> None:
    """Strict mode: wait for every call and raise on a device-side error at once."""
    _state["strict"] = bool(flag)


def _raise_status(code: int) -> None:
    if code == _lib.FRNN_E_PLACEMENT:
        _state["xcd_shared"] = True  # later calls use the placement-free exchange
    raise RuntimeError(f"flashrnn_amd device error: {_lib.strerror(code)} (code {code})")


def _drain_pending(block: bool = False) -> None:
    while _pending:
        host, event = _pending[0]
        if not block and not event.query():
            return
        event.synchronize()
        _pending.popleft()
        v = int(host[0])
        if v:
            _raise_status(-v)


def synchronize_and_check() -> None:
    """Wait for all outstanding calls and raise if any reported a device error."""
    _drain_pending(block=True)


def _after_call(ws: torch.Tensor) -> None:
    if _state["strict"]:
        rc = _lib.load().frnn_status(ws.data_ptr(), torch.cuda.current_stream(ws.device).cuda_stream)
        if rc != _lib.FRNN_OK:
            _raise_status(rc)
        return
    host = torch.empty(1, dtype=torch.int32, pin_memory=True)
    host.copy_(ws[:4].view(torch.int32), non_blocking=True)
    ev = torch.cuda.Event()
    ev.record()
    _pending.append((host, ev))


def _workspace(nbytes: int, device) -> torch.Tensor:
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
    ws[:256].zero_()  # the status word is sticky; it starts clear
    return ws


# --------------------------------------------------------------------- autograd
def _desc(cell, B, T, N, D, io, st, mma, training, opts=(False, None)):
    cut, clipval = opts
    flags = (_lib.FRNN_TRAINING if training else 0) | (_lib.FRNN_XCD_SHARED if _state["xcd_shared"] else 0)
    flags |= (_lib.FRNN_GRAD_CUT if cut else 0) | (_lib.FRNN_GRAD_CLIP if clipval is not None else 0)
    flags |= _lib.FRNN_TEST_UNREADY if _state["test_unready"] else 0
    return _lib.FrnnDesc(_lib.CELLS[cell], B, T, N, D, _IO[io], _IO[st], mma, flags,
                         float(clipval) if clipval is not None else 0.0)


class _FusedRecurrence(torch.autograd.Function):
    """Autograd contract of the reference's FlashRNNFunctionFused
    (``flashrnn/flashrnn/flashrnn.py:697-802``): saves what the backward kernel needs, returns
    gradients for Wx, R, b and the initial state."""

    @staticmethod
    def forward(ctx, wx, R, b, s0, cell, mma, opts, grad):
        _drain_pending()
        lib = _lib.load()
        B, T, _, N, D = wx.shape
        training = grad  # a backward can follow (grad mode on at the call, an input requires grad)
        d = _desc(cell, B, T, N, D, wx.dtype, s0.dtype, mma, training, opts)
        dev = wx.device
        S = CELL_SIZES[cell][3]
        states = torch.empty((S, B, T, N, D), dtype=wx.dtype, device=dev)
        carry = torch.empty((S, B, N, D), dtype=s0.dtype, device=dev)
        ws = _workspace(lib.frnn_workspace_bytes(d, 0), dev)
        save = torch.empty(lib.frnn_workspace_bytes(d, 2), dtype=torch.uint8, device=dev) if training else None
        stream = torch.cuda.current_stream(dev).cuda_stream
        rc = lib.frnn_fwd(
            d, wx.data_ptr(), R.data_ptr(), b.data_ptr(), s0.data_ptr(), states.data_ptr(), carry.data_ptr(),
            save.data_ptr() if save is not None else None, ws.data_ptr(), ws.numel(), stream,
        )
        _lib.check(rc, "frnn_fwd")
        _after_call(ws)
        if training:
            ctx.save_for_backward(R, s0, states, save)
            ctx.meta = (cell, mma, wx.shape, wx.dtype, b.shape, opts)
        return states, carry

    @staticmethod
    def backward(ctx, d_states, d_carry):
        _drain_pending()
        lib = _lib.load()
        R, s0, states, save = ctx.saved_tensors
        cell, mma, wshape, io, bshape, opts = ctx.meta
        B, T, _, N, D = wshape
        d = _desc(cell, B, T, N, D, io, s0.dtype, mma, True, opts)
        dev = R.device
        d_states = d_states.to(io).contiguous() if d_states is not None else None
        d_carry = d_carry.to(s0.dtype).contiguous() if d_carry is not None else None
        dwx = torch.empty(wshape, dtype=io, device=dev)
        dR = torch.empty(R.shape, dtype=io, device=dev)
        db = torch.empty(bshape, dtype=io, device=dev)
        ds0 = torch.empty(s0.shape, dtype=s0.dtype, device=dev)
        ws = _workspace(lib.frnn_workspace_bytes(d, 1), dev)
        stream = torch.cuda.current_stream(dev).cuda_stream
        rc = lib.frnn_bwd(
            d, R.data_ptr(), s0.data_ptr(), states.data_ptr(), save.data_ptr(),
            d_states.data_ptr() if d_states is not None else None,
            d_carry.data_ptr() if d_carry is not None else None,
            dwx.data_ptr(), dR.data_ptr(), db.data_ptr(), ds0.data_ptr(), ws.data_ptr(), ws.numel(), stream,
        )
        _lib.check(rc, "frnn_bwd")
        _after_call(ws)
        return dwx, dR, db, ds0, None, None, None, None


# ----------------------------------------------------------------------- public API
def _check_shapes(cell, Wx, R, b, states):
    gr, gw, gt, S = CELL_SIZES[cell]
    if Wx.ndim != 5:
        raise ValueError("Wx must have layout [B,T,G,N,D]")
    B, T, G, N, D = Wx.shape
    if min(B, T, N, D) < 1:
        raise ValueError("batch, time, heads and width must be positive")
    if G != gw:
        raise ValueError(f"Wx has {G} gates, cell {cell} expects {gw}")
    if tuple(R.shape) != (gr, N, D, D):
        raise ValueError(f"recurrent weights must have layout [G,N,D,P] = {(gr, N, D, D)}")
    if tuple(b.shape) != (gt, N, D):
        raise ValueError(f"bias must have layout [G,N,D] = {(gt, N, D)}")
    if states is not None and tuple(states.shape) != (S, B, 1, N, D):
        raise ValueError(f"initial state must have layout [S,B,1,N,D] = {(S, B, 1, N, D)}")
    if any(t.device != Wx.device for t in (R, b) + (() if states is None else (states,))):
        raise ValueError("all inputs must be on the same device")
    if Wx.device.type != "cuda":
        raise ValueError("flashrnn_amd runs on a ROCm GPU; inputs must be device tensors")


def io_dtype(wx_dtype: torch.dtype, r_dtype: torch.dtype, b_dtype: torch.dtype) -> torch.dtype:
    """The one tensor dtype the kernels run on when Wx, R and b differ.

    The reference's config keeps separate ``dtype_w``, ``dtype_r`` and ``dtype_b``
    (``flashrnn/flashrnn/flashrnn.py:187-264``, ``_get_config`` at ``:1096-1114``) and
    compiles a kernel for that mix. Here all three are promoted to the widest of
    them (FP32 if any is FP32; BF16 and FP16 together promote to FP32), so no
    input loses precision before the policy rounds the recurrent operands; the
    state history is returned in Wx's dtype and each gradient in its input's
    dtype. Unsupported dtypes raise ``ValueError``."""
    for name, dt in (("Wx", wx_dtype), ("R", r_dtype), ("b", b_dtype)):
        if dt not in _IO:
            raise ValueError(f"{name} dtype {dt} not supported; use bfloat16, float16 or float32")
    kinds = {wx_dtype, r_dtype, b_dtype}
    return kinds.pop() if len(kinds) == 1 else torch.float32


def flashrnn(
    Wx: torch.Tensor,
    R: torch.Tensor,
    b: torch.Tensor,
    states: Optional[torch.Tensor] = None,
    function: str = "lstm",
    config: Optional[FlashRNNConfig] = None,
    backend: str = "cuda_fused",
    dtype: str = "bfloat16",
):
    """Fused multi-head recurrence. Returns ``(states [S,B,T,N,D], last [S,B,1,N,D])``."""
    if config is None:
        config = FlashRNNConfig(backend=backend, function=function, dtype=dtype)
    cell = config.function
    # caller-side layouts -> the kernels' [B,T,G,N,D], [G,N,D,P], [G,N,D], [S,B,T,N,D]
    # (the reference's letters: H is the head index N here)
    if config.input_shape != "BTGHD" and Wx.ndim == 5:
        Wx = Wx.permute(_perm(config.input_shape, "BTGHD"))
    if config.recurrent_shape != "GHDP" and R.ndim == 4:
        R = R.permute(_perm(config.recurrent_shape, "GHDP"))
    if config.bias_shape != "GHD" and b.ndim == 3:
        b = b.permute(_perm(config.bias_shape, "GHD"))
    if states is not None and config.output_shape != "SBTHD" and states.ndim == 5:
        states = states.permute(_perm(config.output_shape, "SBTHD"))
    if states is None and config.initial_val != 0.0 and Wx.ndim == 5:
        S, (B, _, _, N, D) = CELL_SIZES[cell][3], Wx.shape
        iv = config.initial_val
        vals = [float(iv)] * S if isinstance(iv, (int, float)) else [float(v) for v in iv]
        states = torch.tensor(vals, dtype=Wx.dtype, device=Wx.device).view(S, 1, 1, 1, 1).expand(S, B, 1, N, D)
    hist, last = _flashrnn(Wx, R, b, states, cell, config)
    if config.output_shape != "SBTHD":
        p = _perm("SBTHD", config.output_shape)
        hist, last = hist.permute(p), last.permute(p)
    return hist, last


def _perm(src: str, dst: str) -> tuple:
    """Dimension order that takes layout ``src`` to ``dst`` (``permute_to``, flashrnn.py:97-108)."""
    return tuple(src.index(x) for x in dst)


def _flashrnn(Wx, R, b, states, cell, config):
    _check_shapes(cell, Wx, R, b, states)
    out_dtype = Wx.dtype
    io = io_dtype(Wx.dtype, R.dtype, b.dtype)
    mma = _MMA[config.dtype]
    B, T, _, N, D = Wx.shape
    S = CELL_SIZES[cell][3]
    if states is None:
        s0 = torch.zeros((S, B, N, D), dtype=io, device=Wx.device)
    else:
        st_dtype = states.dtype if states.dtype in _IO else io
        s0 = states.to(st_dtype)[:, :, 0]
    Wx = Wx.to(io)
    R = R.to(io)
    b = b.to(io)
    # width: the kernels tile hidden units by 32; pad with inert units (zero
    # weights, inputs and states), which never reach a real unit.
    Dp = (D + 31) // 32 * 32
    if Dp > 1024:
        raise ValueError(f"head width {D} exceeds the supported maximum 1024")
    if Dp != D:
        pad = Dp - D
        Wx = F.pad(Wx, (0, pad))
        R = F.pad(R, (0, pad, 0, pad))
        b = F.pad(b, (0, pad))
        s0 = F.pad(s0, (0, pad))
    opts = (bool(config.gradient_recurrent_cut), config.gradient_recurrent_clipval)
    grad = torch.is_grad_enabled() and any(t.requires_grad for t in (Wx, R, b, s0))
    hist, carry = _FusedRecurrence.apply(Wx.contiguous(), R.contiguous(), b.contiguous(), s0.contiguous(), cell, mma,
                                         opts, grad)
    if Dp != D:
        hist = hist[..., :D]
        carry = carry[..., :D]
    return hist.to(out_dtype), carry.unsqueeze(2)

"""Prepared, forward-only sequence execution with fixed buffers and an output policy.

Mirrors FlashRNN2's ``PreparedSequence`` (``flashrnn/flashrnn2/prepared.py:18-192``):
inputs, weights and outputs have fixed device addresses; one instance runs the
whole sequence, optionally in chunks, through ``frnn_fwd`` of ``libfrnn.so``
(the persistent gfx950 recurrence kernels), and can be captured once into a
HIP graph and replayed. Results are borrowed buffers: the next execution
overwrites them. An instance is used serially on one stream; refresh its
input buffers (``wx``, ``initial``, ...) on that stream before ``run()``.

Output policies (``prepared.py:22-23, 71-74``; ``triton_persistent.py:154-166``):

* ``"full"``   -- every state of every step, ``[S,B,T,N,D]``;
* ``"hidden"`` -- the hidden state of every step, ``[B,T,N,D]``;
* ``"last"``   -- the hidden state of the last step, ``[B,1,N,D]``;

in ``snapshot_dtype`` (the input dtype, or FP32). ``final`` is the FP32
compute carry ``[S,B,1,N,D]`` after the last step, whatever the policy.
Chunks (``prepared.py:64-66, 114-162``) run consecutive step windows of the
same buffers; each continues from the previous window's FP32 carry (two carry
buffers alternate), so a chunked run equals the unchunked run bitwise.

Differences from the reference, on purpose: every cell of the fused path is
accepted (the reference's prepared path has LSTM and sLSTM only), Wx has the
cell's own gate count, inputs are BF16 or FP16 (recurrent product with 16-bit
operands, FP32 accumulation and state -- the arithmetic of the reference's
prepared kernels) or FP32 (FP32 product); the head width must be a multiple
of 16 from 16 to 1024 (as the reference requires a multiple of 16; widths that
are not a multiple of 32 run on padded copies that every run refreshes from the
caller's tensors, so in-place updates still reach the next run);
``config`` is this library's :class:`KernelConfig`, not the reference's
kernel-family table (``execution_policy.py:11-60``), which names CUDA
families that do not exist here.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from .flashrnn import _IO, _MMA_OF, CELL_SIZES, _state

_MODES = {"full": 0, "hidden": _lib.FRNN_OUT_HIDDEN, "last": _lib.FRNN_OUT_LAST}


@dataclass(frozen=True)
class KernelConfig:
    """Launch options of the prepared path.

    ``exchange``: ``"xcd"`` keeps every recurrence group on one XCD and
    exchanges hidden states through that XCD's L2 (the fast default);
    ``"shared"`` exchanges through memory-side coherence and accepts any
    workgroup placement (``FRNN_XCD_SHARED``). ``None`` takes the library's
    current choice (shared once a placement error has been seen)."""

    exchange: str | None = None

    def __post_init__(self):
        if self.exchange not in (None, "xcd", "shared"):
            raise ValueError("exchange must be 'xcd', 'shared' or None")


def default_config(width: int | None = None) -> KernelConfig:
    """The configuration used when none is given (``execution_policy.default_config``)."""
    return KernelConfig()


class PreparedSequence:
    """Fixed-buffer forward execution of one recurrence (``prepared.py:18-110``).

    ``wx [B,T,G_W,N,D]``, ``recurrent [G_R,N,D,D]``, ``bias [G_T,N,D]``,
    ``initial [S,B,1,N,D]`` (input dtype or FP32) are kept by reference, not
    copied: later in-place updates of these tensors are what the next
    ``run()`` reads.
    """

    def __init__(self, wx, recurrent, bias, initial, cell="lstm", *,
                 output_mode="full", snapshot_dtype=None, config=None, chunks=None):
        if output_mode not in _MODES:
            raise ValueError("output mode must be full, hidden or last")
        if cell not in CELL_SIZES:
            raise ValueError(f"unknown cell {cell!r}")
        gr, gw, gt, S = CELL_SIZES[cell]
        if wx.ndim != 5:
            raise ValueError(f"expected Wx [B,T,{gw},H,D]")
        batch, steps, gates, heads, width = wx.shape
        if gates != gw or batch < 1 or steps < 1 or heads < 1:
            raise ValueError(f"expected nonempty B/T/H and {gw} gates for {cell}")
        if width % 16 or not 16 <= width <= 1024:
            raise ValueError("prepared execution needs D >= 16, a multiple of 16, at most 1024")
        if recurrent.shape != (gr, heads, width, width) or bias.shape != (gt, heads, width):
            raise ValueError("invalid recurrent-weight or bias shape")
        if initial.shape != (S, batch, 1, heads, width):
            raise ValueError("invalid initial-state shape")
        tensors = (wx, recurrent, bias, initial)
        if wx.dtype not in _IO:
            raise ValueError("inputs must be bfloat16, float16 or float32")
        if recurrent.dtype != wx.dtype or bias.dtype != wx.dtype or initial.dtype not in (wx.dtype, torch.float32):
            raise ValueError("input dtype does not match generic computation contract")
        if any(x.requires_grad for x in tensors):
            raise ValueError("prepared execution is forward-only")
        dtype = wx.dtype if snapshot_dtype is None else snapshot_dtype
        if dtype not in (wx.dtype, torch.float32):
            raise ValueError("snapshot dtype must be input dtype or FP32")
        lengths = (steps,) if chunks is None else tuple(chunks)
        if not lengths or any(type(n) is not int or n < 1 for n in lengths) or sum(lengths) != steps:
            raise ValueError("chunk lengths must be positive integers totaling T")
        if not wx.is_cuda or any(x.device != wx.device or not x.is_contiguous() for x in tensors):
            raise ValueError("prepared execution requires contiguous tensors on one GPU device")
        config = config or default_config(width)
        if not isinstance(config, KernelConfig):
            raise ValueError("config must be a flashrnn_amd.prepared.KernelConfig")

        self.wx, self.recurrent, self.bias, self.initial = tensors
        self.cell, self.shape, self.chunks, self.config = cell, (batch, steps, heads, width), lengths, config
        self.output_mode = output_mode
        dev = wx.device
        shape = (S, batch, steps, heads, width) if output_mode == "full" else (
            batch, 1 if output_mode == "last" else steps, heads, width)
        self.output = torch.empty(shape, dtype=dtype, device=dev)
        # The kernels tile hidden units by 32. A width that is a multiple of 16
        # only runs on zero-padded copies (inert units: zero weights, inputs and
        # states), refreshed from the caller's tensors in every run; the
        # outputs are copied back without the padding.
        kw = width + (-width) % 32
        self._padded = kw != width
        if self._padded:
            pad = lambda t, shp, dt=None: torch.zeros(shp, dtype=dt or t.dtype, device=dev)
            self._wx = pad(wx, (batch, steps, gates, heads, kw))
            self._recurrent = pad(recurrent, (gr, heads, kw, kw))
            self._bias = pad(bias, (gt, heads, kw))
            self._output = pad(self.output, shape[:-1] + (kw,))
        else:
            self._wx, self._recurrent, self._bias, self._output = wx, recurrent, bias, self.output
        # FP32 compute carries, alternating between chunks; an FP32 copy of a
        # lower-precision initial state (exact) is refreshed in every run
        cshape = initial.shape[:-1] + (kw,)
        self.carries = tuple(torch.zeros(cshape, dtype=torch.float32, device=dev) for _ in range(2))
        self.final = self.carries[(len(lengths) - 1) % 2]
        self.initial32 = None if initial.dtype == torch.float32 and not self._padded else torch.zeros(
            cshape, dtype=torch.float32, device=dev)
        if self._padded:
            self.final = torch.empty(initial.shape, dtype=torch.float32, device=dev)

        exchange = config.exchange or ("shared" if _state["xcd_shared"] else "xcd")
        flags = _MODES[output_mode] | (_lib.FRNN_SNAPSHOT_F32 if dtype == torch.float32 else 0)
        flags |= _lib.FRNN_XCD_SHARED if exchange == "shared" else 0
        flags |= _lib.FRNN_TEST_UNREADY if _state["test_unready"] else 0  # failure-handling tests only
        mma = _MMA_OF[wx.dtype]
        lib = _lib.load()
        self._descs, start = [], 0
        for n in lengths:
            d = _lib.FrnnDesc(_lib.CELLS[cell], batch, n, heads, kw, _IO[wx.dtype], _lib.FRNN_F32, mma, flags,
                              0.0, steps, start)
            if lib.frnn_workspace_bytes(d, 0) == 0:
                raise ValueError(f"unsupported prepared configuration {cell} B{batch} T{n} N{heads} D{width}")
            self._descs.append(d)
            start += n
        nbytes = max(lib.frnn_workspace_bytes(d, 0) for d in self._descs)
        self.workspace = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=dev)  # status word starts clear
        self._graph = None

    def _execute(self):
        lib = _lib.load()
        stream = torch.cuda.current_stream(self.wx.device).cuda_stream
        D = self.shape[3]
        if self._padded:
            self._wx[..., :D].copy_(self.wx)
            self._recurrent[..., :D, :D].copy_(self.recurrent)
            self._bias[..., :D].copy_(self.bias)
        previous = self.initial
        if self.initial32 is not None:
            self.initial32[..., :D].copy_(self.initial)
            previous = self.initial32
        ws = self.workspace
        for index, d in enumerate(self._descs):
            carry = self.carries[index % 2]
            rc = lib.frnn_fwd(d, self._wx.data_ptr(), self._recurrent.data_ptr(), self._bias.data_ptr(),
                              previous.data_ptr(), self._output.data_ptr(), carry.data_ptr(), None,
                              ws.data_ptr(), ws.numel(), stream)
            _lib.check(rc, "frnn_fwd")
            previous = carry
        if self._padded:
            self.output.copy_(self._output[..., :D])
            self.final.copy_(previous[..., :D])
        return self.output, self.final

    def check(self):
        """Synchronize and raise if a recurrence exchange reported an error (``prepared.py:164-167``).
        The status word is sticky: once set, every later check raises."""
        rc = _lib.load().frnn_status(self.workspace.data_ptr(),
                                     torch.cuda.current_stream(self.wx.device).cuda_stream)
        if rc != _lib.FRNN_OK:
            raise RuntimeError(f"recurrence exchange failed: {_lib.strerror(rc)}; outputs are invalid")

    def run(self):
        """Execute (or replay the captured graph); returns ``(output, final)``."""
        if self._graph is not None:
            self._graph.replay()
            return self.output, self.final
        return self._execute()

    def capture(self):
        """Capture one execution into a HIP graph after three warm-up executions
        on a side stream (``prepared.py:174-187``)."""
        if self._graph is not None:
            raise ValueError("sequence is already captured")
        with torch.cuda.device(self.wx.device):
            stream = torch.cuda.Stream()
            stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(stream):
                for _ in range(3):
                    self._execute()
            torch.cuda.current_stream().wait_stream(stream)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self._execute()
            self._graph = graph
        return self

    def close(self):
        """Release the captured graph (``prepared.py:189-193``)."""
        if self._graph is not None:
            torch.cuda.synchronize(self.wx.device)
            self._graph.reset()
            self._graph = None

"""frnn_fwd_projected on the GPU: the input projection's workers beside the
recurrence in one launch, against the same workers in a launch of their own
(FRNN_PROJ_OVERLAP=0), against frnn_fwd on the Wx they wrote, and against an
FP32 GEMM of the same 16-bit operands.

* Wx: each element within one unit in the last place of the 16-bit type of the
  FP32 product of the same operands (FP32 accumulation rounded once; the sum's
  order may differ from torch's);
* states, carry and the saved-for-backward area: bitwise equal to frnn_fwd on
  that Wx, and the overlapped launch bitwise equal to the separate one.

Cases: the LSTM at the C2 head shape (B8 N3 D256, 48 recurrence CUs), ragged
batch and time, widths and input sizes that leave partial tiles (I = 8, 40,
136; 32 and 576 columns), workers in workgroups of two, three, five and
eight waves (D = 32, 64, 256, 768), FP16 operands, and a recurrence that
fills every CU (the workers then run in their own launch). The layer at C2 (T1024, I768) is
checked forward and backward against the oracle's projection + flashrnn_torch.
"""

import ctypes
import os

import pytest
import torch

from flashrnn_amd import _lib
from flashrnn_amd.flashrnn import CELL_SIZES

pytestmark = pytest.mark.gpu

MMA = {torch.bfloat16: _lib.FRNN_MMA_BF16, torch.float16: _lib.FRNN_MMA_F16}
IO = {torch.bfloat16: _lib.FRNN_BF16, torch.float16: _lib.FRNN_F16}
ULP = {torch.bfloat16: 2.0**-7, torch.float16: 2.0**-10}


def inputs(cell, B, T, N, D, I, io, seed):
    g = torch.Generator().manual_seed(seed)
    gr, gw, gt, S = CELL_SIZES[cell]
    x = torch.randn(B, T, I, generator=g)
    W = torch.randn(gw, N, D, I, generator=g) / I**0.5
    R = torch.randn(gr, N, D, D, generator=g) / D**0.5
    b = 0.1 * torch.randn(gt, N, D, generator=g)
    s0 = 0.5 * torch.randn(S, B, N, D, generator=g)
    if cell == "slstm":
        b[1] = 3 + 3 * torch.rand(N, D, generator=g)
        s0[2] = s0[2].abs() + 1
    return [t.to(io).cuda() for t in (x, W, R, b)] + [s0.cuda()]


def forward(cell, B, T, N, D, I, io, args, *, projected, overlap=True, training=False, wx_in=None, flags=None):
    lib = _lib.load()
    gr, gw, gt, S = CELL_SIZES[cell]
    x, W, R, b, s0 = args
    full = flags is not None and not (flags & _lib.FRNN_OUT_HIDDEN)
    flags = (_lib.FRNN_OUT_HIDDEN if flags is None else flags) | (_lib.FRNN_TRAINING if training else 0)
    d = _lib.FrnnDesc(_lib.CELLS[cell], B, T, N, D, IO[io], _lib.FRNN_F32, MMA[io], flags, 0.0, 0, 0)
    wx = torch.empty((B, T, gw, N, D), dtype=io, device="cuda") if projected else wx_in
    hist = torch.empty((S, B, T, N, D) if full else (B, T, N, D), dtype=io, device="cuda")
    carry = torch.empty((S, B, N, D), dtype=torch.float32, device="cuda")
    ws = torch.zeros(lib.frnn_workspace_bytes(ctypes.byref(d), 3 if projected else 0), dtype=torch.uint8,
                     device="cuda")
    save = torch.zeros(lib.frnn_workspace_bytes(ctypes.byref(d), 2), dtype=torch.uint8, device="cuda") \
        if training else None
    sp = save.data_ptr() if training else None
    stream = torch.cuda.current_stream().cuda_stream
    if projected:
        os.environ["FRNN_PROJ_OVERLAP"] = "1" if overlap else "0"
        try:
            rc = lib.frnn_fwd_projected(ctypes.byref(d), I, x.data_ptr(), W.data_ptr(), wx.data_ptr(), R.data_ptr(),
                                        b.data_ptr(), s0.data_ptr(), hist.data_ptr(), carry.data_ptr(), sp,
                                        ws.data_ptr(), ws.numel(), stream)
        finally:
            os.environ.pop("FRNN_PROJ_OVERLAP", None)
        what = "frnn_fwd_projected"
    else:
        rc = lib.frnn_fwd(ctypes.byref(d), wx.data_ptr(), R.data_ptr(), b.data_ptr(), s0.data_ptr(),
                          hist.data_ptr(), carry.data_ptr(), sp, ws.data_ptr(), ws.numel(), stream)
        what = "frnn_fwd"
    _lib.check(rc, what)
    _lib.check(lib.frnn_status(ws.data_ptr(), stream), what + " (device status)")
    return wx, hist, carry, save


CASES = [
    # cell, B, T, N, D, I, dtype, training
    ("lstm", 8, 64, 3, 256, 768, torch.bfloat16, True),
    ("gru", 5, 33, 2, 96, 40, torch.bfloat16, False),
    ("elman", 3, 17, 1, 32, 8, torch.bfloat16, True),
    ("slstm", 16, 20, 2, 128, 64, torch.bfloat16, False),
    ("lstm", 24, 50, 2, 64, 136, torch.float16, True),
    ("gru", 16, 40, 1, 768, 256, torch.bfloat16, True),    # two-tile workgroups (eight waves)
    ("lstm", 8, 30, 1, 640, 128, torch.float16, False),
    ("lstm", 128, 16, 4, 128, 64, torch.bfloat16, False),  # 256 recurrence workgroups: a separate launch
]


@pytest.mark.parametrize("cell,B,T,N,D,I,io,training", CASES,
                         ids=[f"{c[0]}-B{c[1]}T{c[2]}N{c[3]}D{c[4]}I{c[5]}-{str(c[6])[6:]}" for c in CASES])
def test_projected_forward(cell, B, T, N, D, I, io, training):
    print(f"\n[projected] {cell} B{B} T{T} N{N} D{D} I{I} {io} training={training}", flush=True)
    args = inputs(cell, B, T, N, D, I, io, seed=71)
    wx, hist, carry, save = forward(cell, B, T, N, D, I, io, args, projected=True, training=training)
    torch.cuda.synchronize()
    # Wx against the FP32 product of the same operands
    x, W = args[0], args[1]
    ref = (x.float().reshape(B * T, I) @ W.float().reshape(-1, I).t()).view(wx.shape)
    err = (wx.float() - ref).abs() - ULP[io] * ref.abs()
    print(f"  Wx: max |err| - ulp*|ref| = {err.max().item():.3e}", flush=True)
    assert err.max().item() <= 1e-6
    # the workers in their own launch: bitwise the same
    wx1, hist1, carry1, save1 = forward(cell, B, T, N, D, I, io, args, projected=True, overlap=False,
                                        training=training)
    # the recurrence alone on that Wx: bitwise the same
    _, hist2, carry2, save2 = forward(cell, B, T, N, D, I, io, args, projected=False, training=training, wx_in=wx)
    torch.cuda.synchronize()
    assert torch.equal(wx, wx1)
    assert torch.equal(hist, hist1) and torch.equal(carry, carry1)
    assert torch.equal(hist, hist2) and torch.equal(carry, carry2)
    if training:
        assert torch.equal(save, save1) and torch.equal(save, save2)


def test_c2_layer_training():
    """The layer at the C2 recurrence (LSTM B8 T1024 N3 D256) with I = N*D = 768, BF16,
    forward and backward against the oracle at the north star's 1e-2."""
    from flashrnn_amd import set_strict
    from flashrnn_amd.layer import FlashRNNLayer
    from tests.test_gpu_layer import check, layer_inputs, oracle

    set_strict(True)
    print("\n[projected] layer lstm B8 T1024 N3 D256 I768 bf16", flush=True)
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    cpu, dh, dl = layer_inputs("lstm", 8, 1024, 3, 256, 768, seed=64, io=torch.bfloat16)
    layer = FlashRNNLayer(*(t.cuda() for t in cpu[1:4]), "lstm", dtype="bfloat16")
    x = cpu[0].cuda().requires_grad_()
    s0 = cpu[4].cuda().requires_grad_()
    h, l = layer(x, s0, overlap=True)  # the projection in the recurrence's launch, also with a backward
    g = torch.autograd.grad((h.float() * dh.cuda()).sum() + (l * dl.cuda()).sum(),
                            (x, layer.input_weight, layer.recurrent, layer.bias, s0))
    torch.cuda.synchronize()
    check((h, l, *g), oracle("lstm", cpu, dh, dl, "fp32_state_bf16_mma"), 1e-2)


@pytest.mark.parametrize("mode", ["shared-exchange", "full-states"])
def test_projected_options(mode):
    """The placement-free exchange (FRNN_XCD_SHARED: device-coherent Wx loads, no
    scouts) and the full-state output policy, LSTM B8 T48 N3 D256 I256: bitwise
    equal to frnn_fwd on the Wx the call wrote, and to the workers' own launch."""
    print(f"\n[projected] {mode}", flush=True)
    cell, B, T, N, D, I, io = "lstm", 8, 48, 3, 256, 256, torch.bfloat16
    flags = (_lib.FRNN_OUT_HIDDEN | _lib.FRNN_XCD_SHARED) if mode == "shared-exchange" else 0
    args = inputs(cell, B, T, N, D, I, io, seed=72)
    wx, hist, carry, _ = forward(cell, B, T, N, D, I, io, args, projected=True, flags=flags)
    wx1, hist1, carry1, _ = forward(cell, B, T, N, D, I, io, args, projected=True, overlap=False, flags=flags)
    _, hist2, carry2, _ = forward(cell, B, T, N, D, I, io, args, projected=False, wx_in=wx, flags=flags)
    torch.cuda.synchronize()
    assert torch.equal(wx, wx1)
    assert torch.equal(hist, hist1) and torch.equal(carry, carry1)
    assert torch.equal(hist, hist2) and torch.equal(carry, carry2)

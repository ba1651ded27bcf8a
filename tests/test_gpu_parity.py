"""GPU parity: the HIP fused recurrence against the CPU oracle (restated flashrnn_torch).

Tolerances, metric max|a-e| / max|e| per tensor:
  * BF16-operand / FP32-state kernel vs numerics="fp32_state_bf16_mma": 1e-2,
    on all states and on the gradients of Wx, R, b and the initial state;
  * FP32 kernel vs numerics="mathematical" in FP32: 1e-4.
The oracle runs on the CPU on the same seeded inputs.
"""

import pytest
import torch

from oracle.torch_restatement import flashrnn_torch

pytestmark = pytest.mark.gpu

SIZES = {"lstm": (4, 4, 4, 2), "slstm": (4, 4, 4, 4), "gru": (3, 3, 4, 1), "elman": (1, 1, 1, 1)}
TOL = {"bfloat16": 1e-2, "float32": 1e-4}


def rel(a, e):
    a, e = a.detach().double().cpu(), e.detach().double().cpu()
    return ((a - e).abs().max() / e.abs().max().clamp_min(1e-30)).item()


def make(cell, B, T, N, D, seed, zero_state=False, slstm_bias=True):
    g = torch.Generator().manual_seed(seed)
    gr, gw, gt, S = SIZES[cell]
    wx = torch.randn(B, T, gw, N, D, generator=g)
    R = torch.randn(gr, N, D, D, generator=g) / D**0.5
    b = 0.1 * torch.randn(gt, N, D, generator=g)
    s0 = torch.zeros(S, B, 1, N, D) if zero_state else 0.5 * torch.randn(S, B, 1, N, D, generator=g)
    if cell == "slstm":
        if slstm_bias:
            b[1] = 3 + 3 * torch.rand(N, D, generator=g)
        if not zero_state:
            s0[2] = s0[2].abs() + 1
    dh = torch.randn(S, B, T, N, D, generator=g)
    dl = torch.randn(S, B, 1, N, D, generator=g)
    return (wx, R, b, s0), dh, dl


def run_pair(cell, B, T, N, D, dtype, io=torch.float32, seed=0, zero_state=False):
    from flashrnn_amd import flashrnn, set_strict

    set_strict(True)
    cpu, dh, dl = make(cell, B, T, N, D, seed, zero_state)
    # the kernel sees io-typed inputs; the oracle sees exactly those values in FP32
    cpu = tuple(t.to(io).float() for t in cpu)
    numerics = "fp32_state_bf16_mma" if dtype == "bfloat16" else "mathematical"
    leaves = [t.clone().requires_grad_() for t in cpu]
    eh, el = flashrnn_torch(*leaves, cell=cell, numerics=numerics)
    eg = torch.autograd.grad((eh * dh).sum() + (el * dl).sum(), leaves)

    gl = [t.to("cuda", io).requires_grad_() for t in cpu]
    gl[3] = cpu[3].to("cuda").requires_grad_()  # FP32 carry in -> FP32 carry out
    ah, al = flashrnn(gl[0], gl[1], gl[2], gl[3], function=cell, dtype=dtype)
    ag = torch.autograd.grad((ah.float() * dh.cuda()).sum() + (al.float() * dl.cuda()).sum(), gl)
    torch.cuda.synchronize()
    return (ah, al, *ag), (eh, el, *eg)


CASES = [
    # cell, B, T, N, D
    ("lstm", 3, 7, 2, 32),
    ("lstm", 8, 64, 3, 256),
    ("lstm", 5, 9, 1, 64),
    ("gru", 3, 7, 2, 64),
    ("gru", 16, 16, 1, 768),
    ("elman", 3, 7, 2, 32),
    ("elman", 16, 16, 1, 768),
    ("slstm", 3, 7, 2, 64),
    ("slstm", 16, 32, 4, 192),
    ("lstm", 8, 12, 1, 640),
    ("slstm", 5, 8, 1, 576),
    # planner classes: 8 forward waves (D >= 512), 8 backward waves from a wide
    # backward operand (G_R*D/32 >= 16, D128), 4 forward waves at D/32 < 4 (D96)
    ("lstm", 5, 9, 1, 512),
    ("gru", 12, 10, 2, 512),
    ("lstm", 16, 11, 2, 128),
    ("slstm", 4, 9, 2, 128),
    ("gru", 9, 8, 2, 96),
    # 8 forward waves at D384, and at D256 with more than 8 batch rows
    ("lstm", 6, 9, 1, 384),
    ("elman", 12, 9, 2, 256),
    # the GRU's reduce-scatter backward with four compute waves per tile, paired polls
    ("gru", 6, 9, 1, 640),
]


@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
@pytest.mark.parametrize("cell,B,T,N,D", CASES, ids=[f"{c[0]}-B{c[1]}T{c[2]}N{c[3]}D{c[4]}" for c in CASES])
def test_parity_fp32_io(cell, B, T, N, D, dtype):
    if dtype == "float32" and D > 512 and cell != "elman":
        pytest.skip("FP32-operand mode holds R^T and dG fragments for D <= 512 only (register budget); "
                    "the library returns FRNN_E_UNSUPPORTED (see test_abi)")
    print(f"\n[parity] {cell} B{B} T{T} N{N} D{D} {dtype}", flush=True)
    actual, expected = run_pair(cell, B, T, N, D, dtype, seed=B * 1000 + D)
    names = ["states", "last", "dWx", "dR", "db", "ds0"]
    errs = {k: rel(a, e) for k, a, e in zip(names, actual, expected)}
    print(errs, flush=True)
    for k, v in errs.items():
        assert v <= TOL[dtype], (k, v, errs)


@pytest.mark.parametrize("cell", ["lstm", "slstm", "gru", "elman"])
def test_parity_bf16_io(cell):
    """BF16 tensors in and out; the oracle sees the same BF16 values in FP32."""
    print(f"\n[parity-bf16io] {cell}", flush=True)
    actual, expected = run_pair(cell, 4, 16, 2, 64, "bfloat16", io=torch.bfloat16, seed=5)
    names = ["states", "last", "dWx", "dR", "db", "ds0"]
    errs = {k: rel(a, e) for k, a, e in zip(names, actual, expected)}
    print(errs, flush=True)
    for k, v in errs.items():
        assert v <= 1e-2, (k, v, errs)


def test_slstm_zero_start():
    actual, expected = run_pair("slstm", 4, 8, 2, 32, "bfloat16", seed=11, zero_state=True)
    for a, e in zip(actual, expected):
        assert rel(a, e) <= 1e-2


def test_odd_width_is_padded():
    actual, expected = run_pair("lstm", 2, 5, 2, 20, "float32", seed=3)
    for a, e in zip(actual, expected):
        assert rel(a, e) <= 1e-4


@pytest.mark.parametrize("cell,B", [("lstm", 8), ("lstm", 16), ("slstm", 16)])
def test_scouts_change_timing_only(cell, B):
    """The backward's L2-prefetch workgroups (scouts) leave every output bitwise unchanged."""
    from flashrnn_amd import _lib, flashrnn, set_strict

    set_strict(True)
    cpu, dh, dl = make(cell, B, 64, 2, 256, seed=5)
    lib = _lib.load()
    outs = []
    try:
        for on in (1, 0):
            lib.frnn_set_scouts(on)
            gl = [t.to("cuda", torch.bfloat16).requires_grad_() for t in cpu]
            ah, al = flashrnn(*gl, function=cell, dtype="bfloat16")
            ag = torch.autograd.grad((ah.float() * dh.cuda()).sum() + (al.float() * dl.cuda()).sum(), gl)
            torch.cuda.synchronize()
            outs.append([t.detach().cpu() for t in (ah, al, *ag)])
    finally:
        lib.frnn_set_scouts(1)
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("cell,B,T,N,D", [("lstm", 8, 64, 3, 256), ("slstm", 5, 40, 2, 128), ("elman", 16, 33, 1, 192),
                                          ("lstm", 3, 7, 2, 64), ("gru", 3, 7, 2, 64), ("gru", 16, 16, 1, 768)])
@pytest.mark.parametrize("s0_f32", [False, True])
def test_dr_gemm_dma_path(cell, B, T, N, D, s0_f32):
    """BF16 inputs take the LDS-DMA dR GEMM (an FP32 s0, and the GRU's FP32 candidate-gate
    cotangents, through rounded BF16 copies): bitwise
    the register-staged GEMM's dR, and within tolerance of the oracle."""
    from flashrnn_amd import _lib, flashrnn, set_strict

    set_strict(True)
    cpu, dh, dl = make(cell, B, T, N, D, seed=11)
    cpu = tuple(t.to(torch.bfloat16).float() for t in cpu)
    leaves = [t.clone().requires_grad_() for t in cpu]
    eh, el = flashrnn_torch(*leaves, cell=cell, numerics="fp32_state_bf16_mma")
    eg = torch.autograd.grad((eh * dh).sum() + (el * dl).sum(), leaves)
    lib = _lib.load()
    grads = []
    try:
        for on in (1, 0):
            lib.frnn_set_gemm_dma(on)
            gl = [t.to("cuda", torch.bfloat16).requires_grad_() for t in cpu]
            if s0_f32:
                gl[3] = cpu[3].to("cuda").requires_grad_()
            ah, al = flashrnn(*gl, function=cell, dtype="bfloat16")
            ag = torch.autograd.grad((ah.float() * dh.cuda()).sum() + (al.float() * dl.cuda()).sum(), gl)
            torch.cuda.synchronize()
            grads.append([t.detach().cpu() for t in ag])
    finally:
        lib.frnn_set_gemm_dma(1)
    for a, b in zip(*grads):
        assert torch.equal(a, b)
    for name, a, e in zip(("dWx", "dR", "db", "ds0"), grads[0], eg):
        assert rel(a, e) <= 1e-2, (name, rel(a, e))

"""GPU parity of the differentiable output-policy call (FlashRNN2's training
``recurrence``, flashrnn/flashrnn2/training.py:91-228) against the oracle's
``training_recurrence`` (v1 gradient convention for sLSTM, grad_reference.py).

Metric and tolerances as in test_gpu_parity: max|a-e|/max|e| per tensor, 1e-2
for BF16 operands vs numerics="fp32_state_bf16_mma", 1e-4 for FP32 vs
"mathematical". Cross-checks between policies are bitwise: the full policy is
flashrnn()'s kernel pair (for cells without the v1 convention the gradients are
identical), and the hidden policy's gradients equal the full policy's with zero
cotangents on the other states.
"""

import pytest
import torch

from oracle.torch_restatement import training_recurrence
from tests.test_gpu_parity import TOL, make, rel

pytestmark = pytest.mark.gpu

NAMES = ["output", "final", "dWx", "dR", "db", "ds0"]


def weights(out_shape, fin_shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(out_shape, generator=g), torch.randn(fin_shape, generator=g)


def gpu(cell, cpu, io, mode, snap, w, wf):
    from flashrnn_amd import set_strict
    from flashrnn_amd.training import recurrence

    set_strict(True)
    leaves = [t.to("cuda", io).requires_grad_() for t in cpu[:3]] + [cpu[3].to("cuda").requires_grad_()]
    out, fin = recurrence(*leaves, cell, output_mode=mode, snapshot_dtype=snap)
    g = torch.autograd.grad((out.float() * w.cuda()).sum() + (fin * wf.cuda()).sum(), leaves)
    torch.cuda.synchronize()
    return (out, fin, *g)


def oracle(cell, cpu, io, mode, w, wf):
    numerics = "fp32_state_bf16_mma" if io == torch.bfloat16 else "mathematical"
    leaves = [t.to(io).float().requires_grad_() for t in cpu[:3]] + [cpu[3].clone().requires_grad_()]
    out, fin = training_recurrence(*leaves, cell=cell, numerics=numerics, output_mode=mode)
    g = torch.autograd.grad((out * w).sum() + (fin * wf).sum(), leaves)
    return (out, fin, *g)


def check(a, e, tol):
    errs = {k: rel(x, y) for k, x, y in zip(NAMES, a, e)}
    print(errs, flush=True)
    for k, v in errs.items():
        assert v <= tol, (k, v, errs)


def shapes(cell, B, T, N, D, mode):
    S = {"lstm": 2, "slstm": 4, "gru": 1, "elman": 1}[cell]
    out = {"full": (S, B, T, N, D), "hidden": (B, T, N, D), "last": (B, 1, N, D)}[mode]
    return out, (S, B, 1, N, D)


CASES = [("lstm", 5, 12, 2, 64), ("gru", 3, 10, 2, 96), ("elman", 6, 9, 1, 32), ("slstm", 4, 14, 2, 128)]
IDS = [f"{c[0]}-B{c[1]}T{c[2]}N{c[3]}D{c[4]}" for c in CASES]


@pytest.mark.parametrize("snap", [None, torch.float32], ids=["snap_io", "snap_f32"])
@pytest.mark.parametrize("mode", ["full", "hidden", "last"])
@pytest.mark.parametrize("cell,B,T,N,D", CASES, ids=IDS)
def test_training_vs_oracle(cell, B, T, N, D, mode, snap):
    print(f"\n[training] {cell} B{B} T{T} N{N} D{D} {mode} snapshot={snap}", flush=True)
    cpu, _, _ = make(cell, B, T, N, D, seed=31)
    w, wf = weights(*shapes(cell, B, T, N, D, mode), seed=32)
    a = gpu(cell, cpu, torch.bfloat16, mode, snap, w, wf)
    assert a[0].dtype == (snap or torch.bfloat16) and a[1].dtype == torch.float32
    check(a, oracle(cell, cpu, torch.bfloat16, mode, w, wf), TOL["bfloat16"])


@pytest.mark.parametrize("cell", ["lstm", "slstm"])
def test_training_fp32(cell):
    print(f"\n[training] fp32 {cell} B5 T10 N2 D64 hidden", flush=True)
    cpu, _, _ = make(cell, 5, 10, 2, 64, seed=33)
    w, wf = weights(*shapes(cell, 5, 10, 2, 64, "hidden"), seed=34)
    check(gpu(cell, cpu, torch.float32, "hidden", None, w, wf), oracle(cell, cpu, torch.float32, "hidden", w, wf),
          TOL["float32"])


def test_slstm_zero_start_and_headline_shape():
    """sLSTM from a zero state (the clamp's tie at the first step) and the C2 head shape."""
    print("\n[training] slstm zero start B16 T24 N2 D192; lstm B8 T64 N3 D256", flush=True)
    cpu, _, _ = make("slstm", 16, 24, 2, 192, seed=35, zero_state=True)
    w, wf = weights(*shapes("slstm", 16, 24, 2, 192, "hidden"), seed=36)
    check(gpu("slstm", cpu, torch.bfloat16, "hidden", None, w, wf),
          oracle("slstm", cpu, torch.bfloat16, "hidden", w, wf), TOL["bfloat16"])
    cpu, _, _ = make("lstm", 8, 64, 3, 256, seed=37)
    w, wf = weights(*shapes("lstm", 8, 64, 3, 256, "hidden"), seed=38)
    check(gpu("lstm", cpu, torch.bfloat16, "hidden", None, w, wf),
          oracle("lstm", cpu, torch.bfloat16, "hidden", w, wf), TOL["bfloat16"])


@pytest.mark.parametrize("cell", ["lstm", "gru", "elman"])
def test_full_policy_is_flashrnn(cell):
    from flashrnn_amd import flashrnn

    print(f"\n[training] full policy vs flashrnn {cell}", flush=True)
    cpu, dh, dl = make(cell, 5, 11, 2, 64, seed=39)
    a = gpu(cell, cpu, torch.bfloat16, "full", None, dh, dl)
    leaves = [t.to("cuda", torch.bfloat16).requires_grad_() for t in cpu[:3]] + [cpu[3].cuda().requires_grad_()]
    h, last = flashrnn(*leaves, function=cell)
    g = torch.autograd.grad((h.float() * dh.cuda()).sum() + (last * dl.cuda()).sum(), leaves)
    for k, x, y in zip(NAMES, a, (h, last, *g)):
        assert torch.equal(x, y), k


@pytest.mark.parametrize("cell", ["lstm", "slstm", "gru"])
def test_hidden_policy_is_full_with_zero_state_cotangents(cell):
    print(f"\n[training] hidden vs full policy {cell}", flush=True)
    B, T, N, D = 4, 13, 2, 64
    cpu, _, _ = make(cell, B, T, N, D, seed=40)
    w, wf = weights(*shapes(cell, B, T, N, D, "hidden"), seed=41)
    wfull = torch.zeros(shapes(cell, B, T, N, D, "full")[0])
    wfull[0] = w
    a = gpu(cell, cpu, torch.bfloat16, "hidden", None, w, wf)
    b = gpu(cell, cpu, torch.bfloat16, "full", None, wfull, wf)
    assert torch.equal(a[0], b[0][0]) and torch.equal(a[1], b[1])
    for k, x, y in zip(NAMES[2:], a[2:], b[2:]):
        assert torch.equal(x, y), k

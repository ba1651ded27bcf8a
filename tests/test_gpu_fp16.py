"""GPU parity of the FP16 operand path (dtype="float16": FP16 inputs and product
operands, FP32 accumulation and state -- FlashRNN2's FP16 contract,
flashrnn/flashrnn2/state_contract.py:21-49) against the oracle's FP16 policy
(the restatement's ``recurrence`` with FP16 operand rounding, pinned in
test_oracle.py against the explicit NumPy backward).

Metric max|a-e|/max|e| per tensor. Tolerance 2e-3: the north star's 1e-2 bound for
16-bit operands, tightened for FP16's 11-bit significand (measured on MI355X:
2e-4 to 7e-4 on every tensor); the values reached are printed.
"""

import pytest
import torch

from oracle.torch_restatement import recurrence as oracle_recurrence
from tests.test_gpu_parity import make, rel

pytestmark = pytest.mark.gpu

TOL = 2e-3
NAMES = ["states", "last", "dWx", "dR", "db", "ds0"]


def oracle(cell, cpu, dh, dl):
    leaves = [t.clone().requires_grad_() for t in cpu]
    h, l = oracle_recurrence(*leaves, cell=cell, mma_dtype=torch.float16, recurrent_mma_dtype=torch.float16)
    g = torch.autograd.grad((h * dh).sum() + (l * dl).sum(), leaves)
    return (h, l, *g)


def f16_inputs(cell, B, T, N, D, seed, zero_state=False):
    cpu, dh, dl = make(cell, B, T, N, D, seed, zero_state)
    # the kernel sees FP16 Wx, R, b and an FP32 initial state; the oracle the same values
    cpu = tuple(t.half().float() for t in cpu[:3]) + (cpu[3],)
    return cpu, dh, dl


def check(a, e):
    errs = {k: rel(x, y) for k, x, y in zip(NAMES, a, e)}
    print(errs, flush=True)
    for k, v in errs.items():
        assert v <= TOL, (k, v, errs)


CASES = [
    ("lstm", 5, 9, 2, 64), ("lstm", 8, 48, 3, 256), ("gru", 3, 7, 2, 64), ("elman", 3, 7, 2, 32),
    ("slstm", 3, 7, 2, 64), ("gru", 16, 12, 1, 768), ("slstm", 16, 24, 2, 192),
    # a backward wave without k-tiles (GRU D32), a two-tile LSTM over two
    # batch slabs, the widest Elman
    ("gru", 4, 6, 1, 32), ("lstm", 17, 5, 1, 640), ("elman", 20, 6, 2, 1024),
]


@pytest.mark.parametrize("cell,B,T,N,D", CASES, ids=[f"{c[0]}-B{c[1]}T{c[2]}N{c[3]}D{c[4]}" for c in CASES])
def test_f16_parity(cell, B, T, N, D):
    from flashrnn_amd import flashrnn, set_strict

    set_strict(True)
    print(f"\n[fp16] {cell} B{B} T{T} N{N} D{D}", flush=True)
    cpu, dh, dl = f16_inputs(cell, B, T, N, D, seed=51)
    gl = [t.to("cuda", torch.float16).requires_grad_() for t in cpu[:3]] + [cpu[3].cuda().requires_grad_()]
    h, l = flashrnn(*gl, function=cell, dtype="float16")
    assert h.dtype == torch.float16 and l.dtype == torch.float32
    g = torch.autograd.grad((h.float() * dh.cuda()).sum() + (l * dl.cuda()).sum(), gl)
    torch.cuda.synchronize()
    assert all(x.dtype == torch.float16 for x in g[:3])
    check((h, l, *g), oracle(cell, cpu, dh, dl))


def test_f16_prepared_and_training():
    """The output-policy entry points with FP16 inputs."""
    from flashrnn_amd import set_strict
    from flashrnn_amd.prepared import PreparedSequence
    from flashrnn_amd.training import recurrence

    set_strict(True)
    print("\n[fp16] prepared hidden chunks + training hidden, lstm B6 T20 N2 D128", flush=True)
    cpu, dh, dl = f16_inputs("lstm", 6, 20, 2, 128, seed=52)
    args = [t.to("cuda", torch.float16).contiguous() for t in cpu[:3]] + [cpu[3].cuda()]
    p = PreparedSequence(*args, "lstm", output_mode="hidden", snapshot_dtype=torch.float32, chunks=[7, 13])
    out, fin = p.run()
    p.check()
    e = oracle("lstm", cpu, dh, dl)
    assert rel(out, e[0][0]) <= TOL and rel(fin, e[1]) <= TOL
    leaves = [t.clone().requires_grad_() for t in args]
    out, fin = recurrence(*leaves, "lstm", output_mode="hidden")
    w = dh[0].cuda()
    g = torch.autograd.grad((out.float() * w).sum() + (fin * dl.cuda()).sum(), leaves)
    dhz = torch.zeros_like(dh)
    dhz[0] = dh[0]
    e = oracle("lstm", cpu, dhz, dl)
    check((out, fin, *g), (e[0][0], e[1], *e[2:]))

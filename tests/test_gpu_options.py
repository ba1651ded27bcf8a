"""GPU parity of the fused backend's options: gradient_recurrent_cut and
gradient_recurrent_clipval (FlashRNNConfig, flashrnn/flashrnn/flashrnn.py:129-133, 357-380).

The oracle is ``flashrnn_torch_fused_options`` (pinned in test_oracle_options.py).
Tolerances as in test_gpu_parity: max|a-e|/max|e| <= 1e-2 for the BF16-operand
kernel vs numerics="fp32_state_bf16_mma", <= 1e-4 for the FP32 kernel vs
"mathematical". The clip value is chosen so that both clamps are active.
"""

import pytest
import torch

from oracle.torch_restatement import flashrnn_torch_fused_options
from tests.test_gpu_parity import TOL, make, rel

pytestmark = pytest.mark.gpu

NAMES = ["states", "last", "dWx", "dR", "db", "ds0"]
MODES = {"cut": dict(gradient_recurrent_cut=True), "clip": dict(gradient_recurrent_clipval=0.2),
         "cut+clip": dict(gradient_recurrent_cut=True, gradient_recurrent_clipval=0.2)}


def run(cell, B, T, N, D, dtype, opts, seed, io=torch.float32):
    from flashrnn_amd import FlashRNNConfig, flashrnn, set_strict

    set_strict(True)
    cpu, dh, dl = make(cell, B, T, N, D, seed)
    cpu = tuple(t.to(io).float() for t in cpu)
    numerics = "fp32_state_bf16_mma" if dtype == "bfloat16" else "mathematical"
    leaves = [t.clone().requires_grad_() for t in cpu]
    eh, el = flashrnn_torch_fused_options(*leaves, cell=cell, numerics=numerics, **opts)
    eg = torch.autograd.grad((eh * dh).sum() + (el * dl).sum(), leaves, allow_unused=True)
    eg = [torch.zeros_like(x) if g is None else g for g, x in zip(eg, leaves)]

    gl = [t.to("cuda", io).requires_grad_() for t in cpu]
    gl[3] = cpu[3].to("cuda").requires_grad_()
    cfg = FlashRNNConfig(function=cell, dtype=dtype, **opts)
    ah, al = flashrnn(gl[0], gl[1], gl[2], gl[3], config=cfg)
    ag = torch.autograd.grad((ah.float() * dh.cuda()).sum() + (al.float() * dl.cuda()).sum(), gl)
    torch.cuda.synchronize()
    return (ah, al, *ag), (eh, el, *eg)


def check(actual, expected, tol):
    errs = {k: rel(a, e) for k, a, e in zip(NAMES, actual, expected)}
    print(errs, flush=True)
    for k, v in errs.items():
        assert v <= tol, (k, v, errs)


@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize("cell", ["lstm", "gru", "elman", "slstm"])
def test_options_vs_oracle(cell, mode, dtype):
    print(f"\n[options] {cell} {mode} {dtype} B5 T9 N2 D64", flush=True)
    a, e = run(cell, 5, 9, 2, 64, dtype, MODES[mode], seed=11)
    if "clip" in mode:
        assert a[0][0].abs().max().item() <= torch.tensor(0.2).item()  # the forward clamp (FP32 bound) holds
        assert e[0][0].abs().max().item() == pytest.approx(0.2)  # and is active
    check(a, e, TOL[dtype])


@pytest.mark.parametrize("mode", list(MODES))
def test_options_headline_shape(mode):
    """The C2 head shape (paired-row exchange path, eight real batch rows)."""
    print(f"\n[options] lstm {mode} B8 T48 N3 D256", flush=True)
    a, e = run("lstm", 8, 48, 3, 256, "bfloat16", MODES[mode], seed=12, io=torch.bfloat16)
    check(a, e, TOL["bfloat16"])


def test_options_wide_head():
    """Two-tile workgroups (D = 768)."""
    print("\n[options] gru cut+clip B16 T12 N1 D768", flush=True)
    a, e = run("gru", 16, 12, 1, 768, "bfloat16", MODES["cut+clip"], seed=13)
    check(a, e, TOL["bfloat16"])


def test_unreached_clip_matches_plain_kernel():
    """A clip value that no value reaches gives the plain kernel's results (GPU vs GPU)."""
    from flashrnn_amd import FlashRNNConfig, flashrnn, set_strict

    set_strict(True)
    print("\n[options] lstm clip=1e30 vs no option", flush=True)
    cpu, dh, dl = make("lstm", 6, 20, 2, 128, seed=14)
    outs = []
    for opts in ({}, dict(gradient_recurrent_clipval=1e30)):
        gl = [t.to("cuda").requires_grad_() for t in cpu]
        h, l = flashrnn(*gl, config=FlashRNNConfig(function="lstm", **opts))
        g = torch.autograd.grad((h.float() * dh.cuda()).sum() + (l.float() * dl.cuda()).sum(), gl)
        outs.append((h, l, *g))
    torch.testing.assert_close(outs[0][0], outs[1][0], atol=0, rtol=0)  # forward bitwise
    torch.testing.assert_close(outs[0][1], outs[1][1], atol=0, rtol=0)
    for k, a, e in zip(NAMES[2:], outs[1][2:], outs[0][2:]):
        assert rel(a, e) <= 1e-5, k  # backward: the clamped sum adds in another order

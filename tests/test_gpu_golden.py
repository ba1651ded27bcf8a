"""GPU parity straight against vectors the reference itself wrote.

The ``bf16mma_*_wide`` fixtures (``tests/golden/make_golden.py``) come from
the reference's ``flashrnn_torch(numerics="fp32_state_bf16_mma")``
(``flashrnn/flashrnn2/torch_backend.py:12-67``). Every input and upstream
cotangent in them is a BF16 value, so the HIP path gets exactly the values the
reference got. They cover heads of 48-96 units (one to three 32-wide MFMA
k-tiles, 48 padded to 64), batches that fill part of a 16-row tile, and one to
three heads, for all four cells. The bound is 1e-2 max-abs-rel on the states,
the last state and all four gradients.
"""

import glob
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
WIDE = sorted(glob.glob(os.path.join(HERE, "golden", "bf16mma_*_wide.npz")))


def rel(a, e):
    a, e = a.detach().double().cpu(), e.detach().double().cpu()
    return ((a - e).abs().max() / e.abs().max().clamp_min(1e-30)).item()


@pytest.mark.parametrize("path", WIDE, ids=[os.path.basename(p)[:-4] for p in WIDE])
def test_kernel_against_reference_vectors(path):
    from flashrnn_amd import flashrnn, set_strict

    set_strict(True)
    z = np.load(path, allow_pickle=False)
    cell = str(z["cell"])
    host = [torch.from_numpy(z[k]) for k in ("wx", "R", "b", "s0")]
    for t in host:  # the fixture's inputs are BF16 values by construction
        assert torch.equal(t.bfloat16().float(), t)
    leaves = [t.to("cuda", torch.bfloat16).requires_grad_() for t in host]
    print(f"golden {os.path.basename(path)}: cell={cell} wx={tuple(host[0].shape)}", flush=True)
    ah, al = flashrnn(*leaves, function=cell, dtype="bfloat16")
    dh = torch.from_numpy(z["d_hist"]).to("cuda", torch.bfloat16)
    dl = torch.from_numpy(z["d_last"]).to("cuda", torch.bfloat16)
    assert ah.shape == dh.shape and al.shape == dl.shape
    ag = torch.autograd.grad((ah, al), leaves, grad_outputs=(dh, dl))
    torch.cuda.synchronize()
    names = ("states", "last", "dWx", "dR", "db", "ds0")
    expect = [torch.from_numpy(z[k]) for k in ("hist", "last", "dwx", "dR", "db", "ds0")]
    errs = {k: rel(a, e) for k, a, e in zip(names, (ah, al, *ag), expect)}
    print("  max-abs-rel:", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    for k, v in errs.items():
        assert v <= 1e-2, (k, v)


def test_wide_fixtures_present():
    assert {os.path.basename(p)[:-4] for p in WIDE} == {f"bf16mma_{c}_wide" for c in ("lstm", "gru", "elman", "slstm")}

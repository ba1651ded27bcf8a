"""Write golden vectors from the reference's own ``flashrnn_torch`` (run in the build container).

This script imports the reference package from ``/root/reference`` (read-only,
never shipped) and writes *data only*: seeded inputs, upstream cotangents and
the reference's outputs and gradients, one ``.npz`` per case, next to this
file. It is used only for the parts of the oracle that no library routine,
closed form or invariant pins bit for bit:

* the ``fp32_state_bf16_mma`` policy (BF16 rounding of operands *and* of the
  per-step R / hidden cotangents) for all four cells;
* the sLSTM cell (global zero-normalizer predicate, ``maximum`` tie rules),
  in the mathematical policy, FP64, for zero, nonzero and mixed normalizers.

Reference entry point: ``flashrnn/flashrnn2/torch_backend.py:12``.
Usage: ``python tests/golden/make_golden.py [/root/reference]``.
"""

from __future__ import annotations

import pathlib
import sys

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent
SIZES = {"lstm": (4, 4, 2), "slstm": (4, 4, 4), "gru": (3, 4, 1), "elman": (1, 1, 1)}


def make_inputs(cell, B, T, N, D, dtype, seed, normalizer="nonzero"):
    gen = torch.Generator().manual_seed(seed)
    gw, gt, S = SIZES[cell]
    wx = torch.randn(B, T, gw, N, D, generator=gen, dtype=torch.float64)
    R = torch.randn(gw, N, D, D, generator=gen, dtype=torch.float64) / D**0.5
    b = 0.1 * torch.randn(gt, N, D, generator=gen, dtype=torch.float64)
    s0 = 0.5 * torch.randn(S, B, 1, N, D, generator=gen, dtype=torch.float64)
    if cell == "slstm":
        b[1] = 3.0 + 3.0 * torch.rand(N, D, generator=gen, dtype=torch.float64)
        if normalizer == "zero":
            s0.zero_()
        elif normalizer == "nonzero":
            s0[2] = s0[2].abs() + 1.0
        else:  # mixed: some normalizers zero, others not -> global predicate false
            s0[2] = s0[2].abs() + 1.0
            s0[2, 0] = 0.0
    tensors = [t.to(dtype) for t in (wx, R, b, s0)]
    d_hist = torch.randn(S, B, T, N, D, generator=gen, dtype=torch.float64).to(dtype)
    d_last = torch.randn(S, B, 1, N, D, generator=gen, dtype=torch.float64).to(dtype)
    return tensors, d_hist, d_last


def run_case(flashrnn_torch, name, cell, numerics, dtype, normalizer="nonzero", B=3, T=6, N=2, D=8, seed=0,
             bf16_exact=False):
    tensors, d_hist, d_last = make_inputs(cell, B, T, N, D, dtype, seed, normalizer)
    if bf16_exact:
        # every input and cotangent representable in BF16, so a BF16-tensor
        # kernel can be checked against the reference's outputs directly
        tensors = [t.bfloat16().to(dtype) for t in tensors]
        d_hist, d_last = d_hist.bfloat16().to(dtype), d_last.bfloat16().to(dtype)
    leaves = [t.clone().requires_grad_() for t in tensors]
    hist, last = flashrnn_torch(*leaves, cell=cell, numerics=numerics)
    grads = torch.autograd.grad((hist * d_hist).sum() + (last * d_last).sum(), leaves)
    out = {
        "cell": np.array(cell), "numerics": np.array(numerics),
        "wx": tensors[0].numpy(), "R": tensors[1].numpy(), "b": tensors[2].numpy(),
        "s0": tensors[3].numpy(), "d_hist": d_hist.numpy(), "d_last": d_last.numpy(),
        "hist": hist.detach().numpy(), "last": last.detach().numpy(),
        "dwx": grads[0].numpy(), "dR": grads[1].numpy(), "db": grads[2].numpy(), "ds0": grads[3].numpy(),
    }
    np.savez_compressed(HERE / f"{name}.npz", **out)
    print("wrote", name)


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sys.path.insert(0, ref)
    from flashrnn.flashrnn2.torch_backend import flashrnn_torch  # noqa: E402

    seed = 20261201
    for k, cell in enumerate(SIZES):
        run_case(flashrnn_torch, f"bf16mma_{cell}", cell, "fp32_state_bf16_mma", torch.float32, seed=seed + k)
    for k, norm in enumerate(("zero", "nonzero", "mixed")):
        run_case(flashrnn_torch, f"math_slstm_{norm}", "slstm", "mathematical", torch.float64,
                 normalizer=norm, seed=seed + 10 + k)
    run_case(flashrnn_torch, "bf16mma_slstm_zero", "slstm", "fp32_state_bf16_mma", torch.float32,
             normalizer="zero", seed=seed + 20)
    # wider heads: several 32-wide MFMA k-tiles, padded widths, batch rows
    # that do not fill a 16-row tile, more than one head
    for k, (cell, B, T, N, D) in enumerate((("lstm", 10, 12, 2, 96), ("gru", 5, 10, 1, 64),
                                            ("elman", 3, 9, 3, 48), ("slstm", 6, 10, 2, 64))):
        run_case(flashrnn_torch, f"bf16mma_{cell}_wide", cell, "fp32_state_bf16_mma", torch.float32,
                 B=B, T=T, N=N, D=D, seed=seed + 30 + k, bf16_exact=True)


if __name__ == "__main__":
    main()

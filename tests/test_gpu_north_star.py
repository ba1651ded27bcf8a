"""GPU parity at the BASELINE configurations themselves, full size.

* Config 2 (the timed workload of bench.py): LSTM B8 T1024 N3 D256, BF16
  tensors, zero initial state, N(0,1) upstream cotangents on every state and on
  the last state, the inputs bench.py draws (same seed). The HIP path against
  the oracle's ``numerics="fp32_state_bf16_mma"`` on the same BF16-rounded
  values, 1e-2 max-abs-rel on states, last state, dWx, dR, db and ds0.
* Config 1: LSTM B4 T64 N1 D64, FP32 operands, forward, against the committed
  torch.nn.LSTM fixture (tests/golden/c1_lstm_fp32.npz) and the oracle's
  ``"mathematical"`` policy, 1e-4 max-abs-rel.

Each test prints its errors (``pytest -s`` shows them).
"""

import os

import numpy as np
import pytest
import torch

from oracle.torch_restatement import flashrnn_torch

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def rel(a, e):
    a, e = a.detach().double().cpu(), e.detach().double().cpu()
    return ((a - e).abs().max() / e.abs().max().clamp_min(1e-30)).item()


def test_config2_full_size_parity():
    import bench
    from flashrnn_amd import flashrnn, set_strict

    set_strict(True)
    (wx, R, b, s0), (dh, dl) = bench.make_inputs(torch, "cpu")
    # the values the kernel sees: BF16 tensors, as bench.py passes them
    vals = [t.bfloat16().float() for t in (wx, R, b, s0)]
    dh, dl = dh.bfloat16().float(), dl.bfloat16().float()
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    leaves = [t.clone().requires_grad_() for t in vals]
    eh, el = flashrnn_torch(*leaves, cell="lstm", numerics="fp32_state_bf16_mma")
    eg = torch.autograd.grad((eh * dh).sum() + (el * dl).sum(), leaves)

    gl = [t.to("cuda", torch.bfloat16).requires_grad_() for t in vals]
    ah, al = flashrnn(*gl, function="lstm", dtype="bfloat16")
    ag = torch.autograd.grad((ah, al), gl, grad_outputs=(dh.cuda().bfloat16(), dl.cuda().bfloat16()))
    torch.cuda.synchronize()
    errs = {k: rel(a, e) for k, a, e in zip(("states", "last", "dWx", "dR", "db", "ds0"), (ah, al, *ag), (eh, el, *eg))}
    print("config 2 (LSTM B8 T1024 N3 D256) max-abs-rel:", {k: f"{v:.2e}" for k, v in errs.items()})
    for k, v in errs.items():
        assert v <= 1e-2, (k, v)


def test_config1_fp32_kernel():
    from flashrnn_amd import flashrnn, set_strict

    set_strict(True)
    z = np.load(os.path.join(HERE, "golden", "c1_lstm_fp32.npz"), allow_pickle=False)
    args = [torch.from_numpy(z[k]) for k in ("wx", "R", "b", "s0")]
    eh, el = torch.from_numpy(z["hist"]), torch.from_numpy(z["last"])
    oh, ol = flashrnn_torch(*args, cell="lstm", numerics="mathematical")
    with torch.no_grad():
        ah, al = flashrnn(*(a.cuda() for a in args), function="lstm", dtype="float32")
    torch.cuda.synchronize()
    errs = {"states/fixture": rel(ah, eh), "last/fixture": rel(al, el), "states/oracle": rel(ah, oh),
            "last/oracle": rel(al, ol)}
    print("config 1 (LSTM FP32 B4 T64 N1 D64) max-abs-rel:", {k: f"{v:.2e}" for k, v in errs.items()})
    for k, v in errs.items():
        assert v <= 1e-4, (k, v)

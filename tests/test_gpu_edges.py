"""GPU parity at edge shapes: one or two steps, one batch row, batches that
span several 16-row slabs, a 16-wide head padded to 32, the GRU at D <= 32
(a backward compute wave without k-tiles), the widest LSTM head
(D=768, two-tile workgroups), and many heads (more groups than XCDs).

Same oracle and bounds as test_gpu_parity.py (1e-2 max-abs-rel for BF16
operands, 1e-4 for FP32 operands, on states, last state and all gradients).
"""

import pytest

from test_gpu_parity import TOL, rel, run_pair

pytestmark = pytest.mark.gpu

EDGES = [
    # cell, B, T, N, D, dtype
    ("lstm", 4, 1, 2, 64, "bfloat16"),
    ("gru", 3, 2, 1, 96, "bfloat16"),
    ("slstm", 2, 1, 2, 64, "float32"),
    ("elman", 1, 9, 2, 128, "bfloat16"),
    ("gru", 1, 7, 1, 128, "float32"),
    ("lstm", 17, 8, 2, 64, "bfloat16"),
    ("slstm", 33, 6, 1, 64, "bfloat16"),
    ("elman", 40, 5, 3, 32, "float32"),
    ("lstm", 3, 10, 5, 16, "bfloat16"),
    ("lstm", 4, 10, 1, 768, "bfloat16"),
    ("lstm", 16, 8, 48, 16, "bfloat16"),
    ("gru", 9, 6, 20, 32, "bfloat16"),
    # the GRU's backward at D <= 32: three k-tiles over four compute waves, so
    # one wave polls nothing (it must still prefetch its next inputs)
    ("gru", 4, 6, 1, 32, "bfloat16"),
    ("gru", 4, 6, 1, 32, "float32"),
    ("gru", 16, 5, 3, 20, "bfloat16"),
    ("gru", 8, 7, 2, 16, "float32"),
]


@pytest.mark.parametrize("cell,B,T,N,D,dtype", EDGES,
                         ids=[f"{c[0]}-B{c[1]}T{c[2]}N{c[3]}D{c[4]}-{c[5]}" for c in EDGES])
def test_edge_shapes(cell, B, T, N, D, dtype):
    print(f"\n[edge] {cell} B{B} T{T} N{N} D{D} {dtype}", flush=True)
    actual, expected = run_pair(cell, B, T, N, D, dtype, seed=7 * B + T + D)
    names = ["states", "last", "dWx", "dR", "db", "ds0"]
    errs = {k: rel(a, e) for k, a, e in zip(names, actual, expected)}
    print(errs, flush=True)
    for k, v in errs.items():
        assert v <= TOL[dtype], (k, v, errs)


def test_unsupported_width_raises_value_error():
    """LSTM D = 1024 has no kernel here: ValueError before anything runs, as the
    reference raises when no configuration fits; the next call works."""
    import torch

    from flashrnn_amd import flashrnn, set_strict
    from test_gpu_parity import make

    set_strict(True)
    cpu, _, _ = make("lstm", 2, 3, 1, 1024, seed=1)
    with pytest.raises(ValueError, match="unsupported"):
        flashrnn(*(t.cuda().bfloat16() for t in cpu), function="lstm", dtype="bfloat16")
    actual, expected = run_pair("lstm", 2, 3, 1, 64, "bfloat16", seed=2)
    for a, e in zip(actual, expected):
        assert rel(a, e) <= TOL["bfloat16"]
    torch.cuda.synchronize()

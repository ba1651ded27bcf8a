"""GPU parity over the reference's own test size grid.

The reference tests every cell of the fused backend on the grid
B in {2, 8, 16, 64}, D in {32, 64, 512, 1024}, T in {1, 3}, N in {1, 2, 4}
(``flashrnn/tests/test_lstm.py:10-47`` and the same grid in test_gru.py,
test_elman.py, test_slstm.py), plus many heads at D 32/64 and a long case
D = 512, T = 1024. A size with no kernel configuration raises ``ValueError``
there and the tests skip it. This file runs B in {2, 64} of that grid for
every cell, BF16 and FP32 operands, many-head sizes, and the long case at
B = 8, against the oracle at the bounds of test_gpu_parity.py. The sizes this
library has no kernel for (D = 1024 for the gated cells, and for FP32
operands also the Elman) must raise ``ValueError``, as in the reference.
"""

import itertools

import pytest

from test_gpu_parity import TOL, rel, run_pair

pytestmark = pytest.mark.gpu

CELLS = ["lstm", "gru", "elman", "slstm"]
GRID = [(c, B, T, N, D, dt) for c, dt, B, D, T, N in itertools.product(
    CELLS, ["bfloat16", "float32"], [2, 64], [32, 64, 512, 1024], [1, 3], [1, 4])
    if not (dt == "float32" and (B == 64 or N == 4))]  # FP32: a quarter of the grid
MANY_HEADS = [(c, B, 3, N, D, "bfloat16") for c in CELLS for B, N, D in ((64, 128, 32), (16, 64, 64), (2, 128, 64))]
LONG = [(c, 8, 1024, 1, 512, "bfloat16") for c in ("lstm", "gru")]


def supported(cell, D, dtype):
    if D <= 512:
        return True
    return cell == "elman" and dtype != "float32" if D == 1024 else dtype != "float32"


@pytest.mark.parametrize("cell,B,T,N,D,dtype", GRID + MANY_HEADS + LONG,
                         ids=[f"{c[0]}-B{c[1]}T{c[2]}N{c[3]}D{c[4]}-{c[5]}" for c in GRID + MANY_HEADS + LONG])
def test_reference_grid(cell, B, T, N, D, dtype):
    print(f"\n[grid] {cell} B{B} T{T} N{N} D{D} {dtype}", flush=True)
    if not supported(cell, D, dtype):
        with pytest.raises(ValueError, match="unsupported"):
            run_pair(cell, B, T, N, D, dtype, seed=B + T + N + D)
        return
    actual, expected = run_pair(cell, B, T, N, D, dtype, seed=B + T + N + D)
    errs = {k: rel(a, e) for k, a, e in zip(("states", "last", "dWx", "dR", "db", "ds0"), actual, expected)}
    print(errs, flush=True)
    for k, v in errs.items():
        assert v <= TOL[dtype], (k, v, errs)

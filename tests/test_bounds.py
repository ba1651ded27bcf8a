"""Host bounds check of the forward recurrence's addressing (CPU only, no GPU).

tests/bounds/fwd_bounds.cpp enumerates every global element and exchange word
the forward kernel touches, with the index functions the kernels call
(flashrnn_amd/csrc/frnn_plan.h) and the plan libfrnn.so builds, and checks
each against its buffer's extent. The cases include the shape of the
chunked-projection run that ended in a GPU memory fault (B256 T1024 N8 D128,
Wx = 2^30 elements = 2 GiB in BF16, four step windows of 256), unchunked and
in the full-state and training policies, and the other configurations.

tests/bounds/proj_bounds.cpp does the same for the input projection's workers
(frnn_fwd_projected): every operand load of both worker kinds, including the
k runs past the input size and the rows / columns past the end, every Wx
store, the readiness counters and the forward's gate reads.
"""

import pathlib
import shutil
import subprocess

import pytest

from flashrnn_amd import _lib

ROOT = pathlib.Path(__file__).resolve().parents[1]
SRC = ROOT / "tests" / "bounds" / "fwd_bounds.cpp"

LSTM, GRU, ELMAN, SLSTM = 0, 1, 2, 3
F32, BF16 = 0, 1
TRAIN, HIDDEN, LAST = 1, 32, 64

CASES = [
    # cell, B, T, N, D, io, flags, total_steps, windows
    (LSTM, 256, 1024, 8, 128, BF16, HIDDEN, 1024, 4),   # the faulting pipeline's recurrence windows
    (LSTM, 256, 1024, 8, 128, BF16, HIDDEN, 1024, 1),
    (LSTM, 256, 1024, 8, 128, BF16, 0, 1024, 4),        # full-state policy, windows
    (LSTM, 256, 1024, 8, 128, BF16, LAST, 1024, 4),
    (LSTM, 256, 1024, 8, 128, BF16, TRAIN, 1024, 1),    # C5 training forward
    (LSTM, 8, 1024, 3, 256, BF16, TRAIN, 1024, 1),      # C2
    (LSTM, 4, 64, 1, 64, F32, 0, 64, 1),                # C1
    (GRU, 16, 512, 1, 768, BF16, TRAIN, 512, 1),        # C3, two-tile workgroups
    (ELMAN, 16, 512, 1, 768, BF16, TRAIN, 512, 1),
    (SLSTM, 16, 2048, 4, 192, BF16, TRAIN, 2048, 1),    # C4
    (SLSTM, 16, 2048, 4, 192, BF16, HIDDEN, 2048, 8),
    (LSTM, 37, 96, 5, 96, F32, TRAIN, 96, 1),           # ragged batch, odd head count
    (ELMAN, 1000, 48, 3, 1024, BF16, HIDDEN, 48, 3),    # widest head, many slabs
]


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    if not _lib.LIB_PATH.exists():
        pytest.skip("libfrnn.so is not built (python -m flashrnn_amd.build)")
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    exe = tmp_path_factory.mktemp("bounds") / "fwd_bounds"
    lib_dir = str(_lib.LIB_PATH.parent)
    subprocess.run([gxx, "-O2", "-std=c++17", str(SRC), "-o", str(exe), f"-L{lib_dir}", "-lfrnn",
                    f"-Wl,-rpath,{lib_dir}"], check=True)
    return exe


@pytest.mark.parametrize("case", CASES, ids=["cell{}-B{}T{}N{}D{}-io{}-f{}-tt{}-w{}".format(*c) for c in CASES])
def test_forward_addressing_in_bounds(checker, case):
    res = subprocess.run([str(checker), *map(str, case)], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout[-3000:] + res.stderr[-2000:]
    assert res.stdout.strip().endswith("violations 0")


PROJ_SRC = ROOT / "tests" / "bounds" / "proj_bounds.cpp"
PROJ_CASES = [
    # cell, B, T, N, D, io, I
    (LSTM, 8, 1024, 3, 256, BF16, 768),    # the layer at C2
    (GRU, 5, 33, 2, 96, BF16, 40),         # ragged rows and k, 576 columns
    (ELMAN, 3, 17, 1, 32, BF16, 8),        # one partial column tile, I = 8
    (LSTM, 24, 50, 2, 64, 2, 136),         # FP16
    (GRU, 16, 40, 1, 768, BF16, 256),
    (LSTM, 256, 64, 8, 128, BF16, 1024),   # wide input, many row tiles
]


@pytest.fixture(scope="module")
def proj_checker(tmp_path_factory):
    if not _lib.LIB_PATH.exists():
        pytest.skip("libfrnn.so is not built (python -m flashrnn_amd.build)")
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    exe = tmp_path_factory.mktemp("bounds") / "proj_bounds"
    lib_dir = str(_lib.LIB_PATH.parent)
    subprocess.run([gxx, "-O2", "-std=c++17", str(PROJ_SRC), "-o", str(exe), f"-L{lib_dir}", "-lfrnn",
                    f"-Wl,-rpath,{lib_dir}"], check=True)
    return exe


@pytest.mark.parametrize("case", PROJ_CASES, ids=["cell{}-B{}T{}N{}D{}-io{}-I{}".format(*c) for c in PROJ_CASES])
def test_projection_addressing_in_bounds(proj_checker, case):
    res = subprocess.run([str(proj_checker), *map(str, case)], capture_output=True, text=True, timeout=300)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "violations 0" in res.stdout

"""The C ABI of libfrnn.so and the host-side contract, without a GPU.

Covers: every function include/frnn.h declares is exported and bound; cell
gate/state counts equal the reference's registry (flashrnn/flashrnn/flashrnn.py:45-70);
plan and workspace sizing; argument validation that returns before any device
call; and the Python front end's shape/config errors (flashrnn/flashrnn/flashrnn.py
FlashRNNConfig and flashrnn()).
"""

import ctypes
import pathlib
import re

import pytest
import torch

from flashrnn_amd import _lib
from flashrnn_amd.flashrnn import CELL_SIZES, FlashRNNConfig, flashrnn
from oracle.torch_restatement import SIZES as ORACLE_SIZES

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "frnn.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(frnn_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def desc(cell="lstm", B=8, T=1024, N=3, D=256, io=_lib.FRNN_BF16, st=_lib.FRNN_F32, mma=_lib.FRNN_MMA_BF16,
         flags=_lib.FRNN_TRAINING, clipval=0.0):
    return _lib.FrnnDesc(_lib.CELLS[cell], B, T, N, D, io, st, mma, flags, clipval)


def test_header_declares_the_bound_exports():
    assert declared_functions() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name


@pytest.mark.parametrize("cell", ["lstm", "gru", "elman", "slstm"])
def test_cell_sizes_match_reference_registry(lib, cell):
    out = [ctypes.c_int32() for _ in range(4)]
    assert lib.frnn_cell_sizes(_lib.CELLS[cell], *[ctypes.byref(o) for o in out]) == _lib.FRNN_OK
    assert tuple(o.value for o in out) == CELL_SIZES[cell]
    assert CELL_SIZES[cell][1:] == ORACLE_SIZES[cell]


def test_cell_sizes_rejects_unknown_cell(lib):
    out = [ctypes.c_int32() for _ in range(4)]
    assert lib.frnn_cell_sizes(17, *[ctypes.byref(o) for o in out]) == -1


def test_workspace_sizes(lib):
    d = desc()
    ws_f, ws_b, save = (lib.frnn_workspace_bytes(ctypes.byref(d), w) for w in range(3))
    assert ws_f > 0 and ws_b > 0 and save > 0
    # the saved activations grow linearly in T; the exchange workspace does not depend on T
    d2 = desc(T=2048)
    assert lib.frnn_workspace_bytes(ctypes.byref(d2), 2) == 2 * save
    assert lib.frnn_workspace_bytes(ctypes.byref(d2), 0) == ws_f
    # saved activations hold at least one FP32 value per real element and step
    assert save >= 8 * 1024 * 3 * 256 * 4
    assert lib.frnn_workspace_bytes(ctypes.byref(d), 7) == 0


@pytest.mark.parametrize(
    "kw",
    [dict(B=0), dict(T=0), dict(N=0), dict(D=0), dict(io=5), dict(st=9), dict(mma=4)],
)
def test_invalid_descriptors(lib, kw):
    d = desc(**kw)
    assert lib.frnn_workspace_bytes(ctypes.byref(d), 0) == 0
    assert lib.frnn_fwd(ctypes.byref(d), *([None] * 8), 0, None) == -1


@pytest.mark.parametrize("D", [20, 1056, 2048])
def test_unsupported_widths(lib, D):
    d = desc(D=D)
    assert lib.frnn_workspace_bytes(ctypes.byref(d), 0) == 0
    assert lib.frnn_fwd(ctypes.byref(d), *([None] * 8), 0, None) == -2


@pytest.mark.parametrize(
    "cell,D,mma,ok",
    [
        ("lstm", 512, "bf16", True), ("gru", 768, "bf16", True), ("lstm", 768, "bf16", True),
        ("slstm", 576, "bf16", True), ("elman", 1024, "bf16", True), ("gru", 800, "bf16", False),
        ("lstm", 1024, "bf16", False), ("lstm", 512, "f32", True), ("gru", 768, "f32", False),
        ("elman", 768, "f32", True), ("lstm", 768, "f16", True), ("slstm", 256, "f16", True),
        ("lstm", 1024, "f16", False), ("elman", 1024, "f32", False), ("gru", 1024, "bf16", False),
        ("slstm", 1024, "bf16", False),
    ],
)
def test_width_support(lib, cell, D, mma, ok):
    """The plan's register budget: which head widths each operand type supports."""
    m = {"bf16": _lib.FRNN_MMA_BF16, "f16": _lib.FRNN_MMA_F16, "f32": _lib.FRNN_MMA_F32}[mma]
    d = desc(cell=cell, B=16, T=8, N=1, D=D, mma=m)
    assert (lib.frnn_workspace_bytes(ctypes.byref(d), 0) > 0) == ok


@pytest.mark.parametrize(
    "flags,clipval,ok",
    [
        (_lib.FRNN_GRAD_CUT, 0.0, True), (_lib.FRNN_GRAD_CLIP, 0.25, True), (_lib.FRNN_GRAD_CLIP, 0.0, True),
        (_lib.FRNN_GRAD_CUT | _lib.FRNN_GRAD_CLIP, 1.0, True), (_lib.FRNN_GRAD_CLIP, -0.5, False),
        (_lib.FRNN_GRAD_CLIP, float("nan"), False), (_lib.FRNN_GRAD_CLIP, float("inf"), False),
        (1024, 0.0, False), (0, -3.0, True),  # without FRNN_GRAD_CLIP the value is ignored
    ],
)
def test_option_flags(lib, flags, clipval, ok):
    """gradient_recurrent_cut / gradient_recurrent_clipval in the descriptor."""
    d = desc(flags=_lib.FRNN_TRAINING | flags, clipval=clipval)
    assert (lib.frnn_workspace_bytes(ctypes.byref(d), 0) > 0) == ok
    if not ok:
        assert lib.frnn_fwd(ctypes.byref(d), *([None] * 8), 0, None) == -1


@pytest.mark.parametrize(
    "flags,total,base,ok",
    [
        (0, 0, 0, True), (_lib.FRNN_OUT_HIDDEN, 0, 0, True), (_lib.FRNN_OUT_LAST, 0, 0, True),
        (_lib.FRNN_SNAPSHOT_F32, 0, 0, True), (_lib.FRNN_OUT_HIDDEN | _lib.FRNN_SNAPSHOT_F32, 0, 0, True),
        (_lib.FRNN_OUT_HIDDEN | _lib.FRNN_OUT_LAST, 0, 0, False),  # one policy at a time
        (0, 12, 4, True), (0, 12, 8, True), (0, 12, 9, False), (0, 12, -1, False), (0, 3, 0, False),
        (_lib.FRNN_TRAINING | _lib.FRNN_OUT_HIDDEN, 0, 0, True),  # the backward needs the h history only
        (_lib.FRNN_TRAINING | _lib.FRNN_SNAPSHOT_F32, 0, 0, True),
        (_lib.FRNN_TRAINING | _lib.FRNN_OUT_LAST, 0, 0, False),  # forward-only policy
        (_lib.FRNN_TRAINING | _lib.FRNN_SLSTM_V1GRAD, 0, 0, True),
        (_lib.FRNN_TRAINING, 12, 0, False),  # training needs the whole sequence
    ],
)
def test_output_policy_and_window(lib, flags, total, base, ok):
    """Output policies (full / hidden / last, FP32 snapshot) and the forward step window."""
    d = desc(T=4, flags=flags)
    d.total_steps, d.step_base = total, base
    assert (lib.frnn_workspace_bytes(ctypes.byref(d), 0) > 0) == ok
    if ok:
        # the backward rejects its invalid pointers, or a forward-only option before them
        assert lib.frnn_bwd(ctypes.byref(d), *([None] * 11), 0, None) == -1


def test_null_pointers_rejected_before_launch(lib):
    d = desc(B=2, T=4, N=1, D=64)
    assert lib.frnn_fwd(ctypes.byref(d), *([None] * 8), 0, None) == -1
    assert lib.frnn_bwd(ctypes.byref(d), *([None] * 11), 0, None) == -1
    assert lib.frnn_status(None, None) == -1


def test_projected_workspace_and_validation(lib):
    """frnn_fwd_projected: its workspace is the forward's plus one counter per 128-row
    tile (128 rows) of Wx and a tile counter; every argument error returns before a device call
    (the pointers below are never dereferenced)."""
    d = desc(B=8, T=1024, N=3, D=256, flags=0)
    ws_f = lib.frnn_workspace_bytes(ctypes.byref(d), 0)
    ws_p = lib.frnn_workspace_bytes(ctypes.byref(d), 3)
    assert ws_p >= ws_f + 4 * (8 * 1024 // 128 + 1)
    big = 1 << 40
    ok = [0x10000, 0x20000, 0x30000]  # x, w_in, wx_out: 16-byte aligned stand-ins
    rest = [0x40000] * 6               # R, b, s0, states, carry, save

    def call(dd, I, ptrs, ws=0x50000, ws_bytes=big):
        return lib.frnn_fwd_projected(ctypes.byref(dd), I, *ptrs, *rest, ws, ws_bytes, None)

    assert call(d, 64, [None] + ok[1:]) == _lib.FRNN_E_INVALID
    assert call(d, 64, ok, ws=None) == _lib.FRNN_E_INVALID
    assert call(d, 64, [ok[0] + 8] + ok[1:]) == _lib.FRNN_E_INVALID        # misaligned x
    assert call(d, 12, ok) == _lib.FRNN_E_UNSUPPORTED                       # input size not a multiple of 8
    assert call(d, 0, ok) == _lib.FRNN_E_UNSUPPORTED
    d32 = desc(B=8, T=64, N=1, D=64, io=_lib.FRNN_F32, mma=_lib.FRNN_MMA_F32, flags=0)
    assert call(d32, 64, ok) == _lib.FRNN_E_UNSUPPORTED                     # FP32 operands
    dmix = desc(B=8, T=64, N=1, D=64, io=_lib.FRNN_F16, mma=_lib.FRNN_MMA_BF16, flags=0)
    assert call(dmix, 64, ok) == _lib.FRNN_E_UNSUPPORTED                    # operands not in the MMA type
    dwin = _lib.FrnnDesc(_lib.CELLS["lstm"], 8, 32, 1, 64, _lib.FRNN_BF16, _lib.FRNN_F32, _lib.FRNN_MMA_BF16, 0,
                         0.0, 64, 0)
    assert call(dwin, 64, ok) == _lib.FRNN_E_UNSUPPORTED                    # a step window
    assert call(d, 64, ok, ws_bytes=ws_p - 1) == _lib.FRNN_E_WORKSPACE


def test_strerror_names_every_code(lib):
    seen = set()
    for code in range(0, -7, -1):
        s = lib.frnn_strerror(code)
        assert s and s not in seen
        seen.add(s)


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="no fallback"):
        _lib.load(tmp_path / "libfrnn.so")


# ----------------------------------------------------------------- Python front end
def test_config_validation():
    with pytest.raises(ValueError):
        FlashRNNConfig(function="transformer")
    with pytest.raises(ValueError):
        FlashRNNConfig(backend="vanilla")
    with pytest.raises(ValueError):
        FlashRNNConfig(dtype="float64")
    FlashRNNConfig(dtype="float16")
    for bad in (-1.0, float("nan"), float("inf")):
        with pytest.raises(ValueError, match="clipval"):
            FlashRNNConfig(gradient_recurrent_clipval=bad)
    FlashRNNConfig(gradient_recurrent_clipval=0.5, gradient_recurrent_cut=True, forward_clipval=3.0)
    c = FlashRNNConfig(function="slstm")
    assert (c.num_gates_r, c.num_gates_w, c.num_gates_t, c.num_states) == (4, 4, 4, 4)


def test_shape_errors_and_cpu_tensors():
    B, T, N, D = 2, 3, 1, 32
    wx = torch.zeros(B, T, 4, N, D)
    R = torch.zeros(4, N, D, D)
    b = torch.zeros(4, N, D)
    s0 = torch.zeros(2, B, 1, N, D)
    with pytest.raises(ValueError, match="gates"):
        flashrnn(wx[:, :, :3], R, b, s0, function="lstm")
    with pytest.raises(ValueError, match="recurrent weights"):
        flashrnn(wx, R[:, :, :, :16], b, s0, function="lstm")
    with pytest.raises(ValueError, match="bias"):
        flashrnn(wx, R, b[:3], s0, function="lstm")
    with pytest.raises(ValueError, match="initial state"):
        flashrnn(wx, R, b, s0[:1], function="lstm")
    with pytest.raises(ValueError, match="device tensors"):
        flashrnn(wx, R, b, s0, function="lstm")


def test_unsupported_configuration_is_a_value_error():
    """The reference raises ValueError when no kernel configuration fits (its tests
    skip such sizes on it); here FRNN_E_UNSUPPORTED does the same, and stays a
    RuntimeError like every other failed call."""
    with pytest.raises(ValueError, match="unsupported"):
        _lib.check(_lib.FRNN_E_UNSUPPORTED, "frnn_fwd")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.FRNN_E_UNSUPPORTED, "frnn_fwd")
    with pytest.raises(RuntimeError) as e:
        _lib.check(_lib.FRNN_E_TIMEOUT, "frnn_fwd")
    assert not isinstance(e.value, ValueError)

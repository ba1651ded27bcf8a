"""ctypes binding of libfrnn.so (the C ABI declared in include/frnn.h).

The library is built ahead of time (``python -m flashrnn_amd.build``) into
this package directory. Loading fails loudly when it is missing: there is no
fallback path.
"""

from __future__ import annotations

import ctypes
import os
import pathlib

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libfrnn.so"

FRNN_LSTM, FRNN_GRU, FRNN_ELMAN, FRNN_SLSTM = 0, 1, 2, 3
FRNN_F32, FRNN_BF16, FRNN_F16 = 0, 1, 2
FRNN_MMA_BF16, FRNN_MMA_F32, FRNN_MMA_F16 = 0, 1, 2
FRNN_TRAINING, FRNN_XCD_SHARED, FRNN_GRAD_CUT, FRNN_GRAD_CLIP, FRNN_TEST_UNREADY = 1, 2, 4, 8, 16
FRNN_OUT_HIDDEN, FRNN_OUT_LAST, FRNN_SNAPSHOT_F32, FRNN_SLSTM_V1GRAD = 32, 64, 128, 256
FRNN_OK = 0
FRNN_E_INVALID, FRNN_E_UNSUPPORTED, FRNN_E_WORKSPACE, FRNN_E_LAUNCH = -1, -2, -3, -4
FRNN_E_TIMEOUT = -5
FRNN_E_PLACEMENT = -6
FRNN_E_SCRATCH = -7

CELLS = {"lstm": FRNN_LSTM, "gru": FRNN_GRU, "elman": FRNN_ELMAN, "slstm": FRNN_SLSTM}


class FrnnDesc(ctypes.Structure):
    _fields_ = [
        ("cell", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("steps", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("width", ctypes.c_int32),
        ("dtype_io", ctypes.c_int32),
        ("dtype_state", ctypes.c_int32),
        ("mma", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("clipval", ctypes.c_float),
        ("total_steps", ctypes.c_int32),
        ("step_base", ctypes.c_int32),
    ]


EXPORTS = (
    "frnn_cell_sizes",
    "frnn_workspace_bytes",
    "frnn_fwd",
    "frnn_fwd_projected",
    "frnn_fwd_noalloc",
    "frnn_bwd",
    "frnn_status",
    "frnn_strerror",
    "frnn_set_spin_limit",
    "frnn_set_scouts",
    "frnn_set_gemm_dma",
    "frnn_timing_enable",
    "frnn_timing_read",
    "frnn_set_phase_profile",
)

_lib = None


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load libfrnn.so once and declare its signatures."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = pathlib.Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"libfrnn.so not found at {p}; build it with `python -m flashrnn_amd.build` "
            "(there is no fallback implementation)"
        )
    lib = ctypes.CDLL(str(p))
    vp, sz, i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
    dp = ctypes.POINTER(FrnnDesc)
    lib.frnn_cell_sizes.argtypes = [i32] + [ctypes.POINTER(ctypes.c_int32)] * 4
    lib.frnn_cell_sizes.restype = i32
    lib.frnn_workspace_bytes.argtypes = [dp, i32]
    lib.frnn_workspace_bytes.restype = sz
    lib.frnn_fwd.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
    lib.frnn_fwd.restype = i32
    lib.frnn_fwd_projected.argtypes = [dp, ctypes.c_int32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
    lib.frnn_fwd_projected.restype = i32
    lib.frnn_fwd_noalloc.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.frnn_fwd_noalloc.restype = i32
    lib.frnn_bwd.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
    lib.frnn_bwd.restype = i32
    lib.frnn_status.argtypes = [vp, vp]
    lib.frnn_status.restype = i32
    lib.frnn_strerror.argtypes = [i32]
    lib.frnn_strerror.restype = ctypes.c_char_p
    lib.frnn_set_spin_limit.argtypes = [ctypes.c_uint32]
    lib.frnn_set_spin_limit.restype = None
    lib.frnn_set_scouts.argtypes = [i32]
    lib.frnn_set_scouts.restype = None
    lib.frnn_set_gemm_dma.argtypes = [i32]
    lib.frnn_set_gemm_dma.restype = None
    lib.frnn_timing_enable.argtypes = [i32]
    lib.frnn_timing_enable.restype = None
    lib.frnn_timing_read.argtypes = [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int32)]
    lib.frnn_timing_read.restype = i32
    lib.frnn_set_phase_profile.argtypes = [vp]
    lib.frnn_set_phase_profile.restype = None
    if path is None:
        _lib = lib
    return lib


def timing_read() -> tuple[list[float], list[int]]:
    """Summed milliseconds and launch counts: [forward recurrence, backward recurrence, dR GEMM]."""
    ms = (ctypes.c_double * 3)()
    cnt = (ctypes.c_int32 * 3)()
    check(load().frnn_timing_read(ms, cnt), "frnn_timing_read")
    return list(ms), list(cnt)


def strerror(code: int) -> str:
    return load().frnn_strerror(code).decode()


class UnsupportedConfiguration(ValueError, RuntimeError):
    """A shape, width or option mix the library has no kernel for.

    A ``ValueError``, as the reference raises when no kernel configuration
    solves its constraints (``flashrnn/flashrnn/cuda_init_parametric.py:25-65``;
    its tests skip such sizes on ``ValueError``), and a ``RuntimeError`` like
    every other failed call here."""


def check(code: int, what: str) -> None:
    if code == FRNN_E_UNSUPPORTED:
        raise UnsupportedConfiguration(f"{what} failed: {strerror(code)} (code {code})")
    if code != FRNN_OK:
        raise RuntimeError(f"{what} failed: {strerror(code)} (code {code})")

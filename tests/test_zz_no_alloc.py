"""frnn_fwd_noalloc (the allocation-free forward) against frnn_fwd, through the C ABI.

Two calls in a row on the same GPU, the second with a smaller problem (the
static scratch keeps the first call's contents), each bitwise equal to
frnn_fwd on the same inputs with a workspace of its own; a problem beyond the
scratch maximum is refused with FRNN_E_SCRATCH before anything runs.
"""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _desc(lib_mod, cell, B, T, N, D, flags=0):
    io = lib_mod.FRNN_BF16
    return lib_mod.FrnnDesc(lib_mod.CELLS[cell], B, T, N, D, io, lib_mod.FRNN_F32, lib_mod.FRNN_MMA_BF16, flags,
                            0.0, 0, 0)


def _inputs(cell, B, T, N, D, seed):
    sizes = {"lstm": (4, 4, 4, 2), "gru": (3, 3, 4, 1), "elman": (1, 1, 1, 1), "slstm": (4, 4, 4, 4)}
    gr, gw, gt, S = sizes[cell]
    g = torch.Generator().manual_seed(seed)
    wx = torch.randn(B, T, gw, N, D, generator=g).bfloat16().cuda()
    R = (torch.randn(gr, N, D, D, generator=g) / D**0.5).bfloat16().cuda()
    b = (0.1 * torch.randn(gt, N, D, generator=g)).bfloat16().cuda()
    s0 = (0.5 * torch.randn(S, B, N, D, generator=g)).cuda()
    if cell == "slstm":
        s0[2] = s0[2].abs() + 1
    return wx, R, b, s0, S


def _run(lib, d, cell, B, T, N, D, wx, R, b, s0, S, noalloc, training):
    states = torch.full((S, B, T, N, D), float("nan"), dtype=torch.bfloat16, device="cuda")
    carry = torch.full((S, B, N, D), float("nan"), device="cuda")
    save = None
    if training:
        save = torch.zeros(lib.frnn_workspace_bytes(ctypes.byref(d), 2), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    args = [ctypes.byref(d), wx.data_ptr(), R.data_ptr(), b.data_ptr(), s0.data_ptr(), states.data_ptr(),
            carry.data_ptr(), save.data_ptr() if save is not None else None]
    if noalloc:
        status = torch.zeros(1, dtype=torch.int32, device="cuda")
        rc = lib.frnn_fwd_noalloc(*args, status.data_ptr(), stream)
        word = status
    else:
        ws = torch.zeros(lib.frnn_workspace_bytes(ctypes.byref(d), 0), dtype=torch.uint8, device="cuda")
        rc = lib.frnn_fwd(*args, ws.data_ptr(), ws.numel(), stream)
        word = ws[:4].view(torch.int32)
    assert rc == 0, rc
    torch.cuda.synchronize()
    assert int(word.item()) == 0
    return states, carry, save


# (cell, B, T, N, D, training): the second case of each pair is smaller than the first
PAIRS = [
    (("lstm", 8, 64, 3, 256, False), ("lstm", 3, 9, 2, 64, False)),
    (("gru", 16, 32, 2, 768, True), ("gru", 5, 7, 1, 128, True)),
    (("slstm", 20, 24, 2, 192, False), ("elman", 4, 6, 1, 32, False)),
]


@pytest.mark.parametrize("first,second", PAIRS, ids=[f"{p[0][0]}-then-{p[1][0]}" for p in PAIRS])
def test_noalloc_equals_frnn_fwd(first, second):
    from flashrnn_amd import _lib

    lib = _lib.load()
    for k, (cell, B, T, N, D, training) in enumerate((first, second)):
        print(f"noalloc case {k}: {cell} B{B} T{T} N{N} D{D} training={training}", flush=True)
        d = _desc(_lib, cell, B, T, N, D, _lib.FRNN_TRAINING if training else 0)
        wx, R, b, s0, S = _inputs(cell, B, T, N, D, seed=17 + k)
        ref = _run(lib, d, cell, B, T, N, D, wx, R, b, s0, S, noalloc=False, training=training)
        got = _run(lib, d, cell, B, T, N, D, wx, R, b, s0, S, noalloc=True, training=training)
        for name, a, e in zip(("states", "carry", "save"), got, ref):
            if e is None:
                continue
            assert torch.equal(a.view(torch.uint8) if a.dtype != torch.uint8 else a,
                               e.view(torch.uint8) if e.dtype != torch.uint8 else e), name


def test_noalloc_rejects_oversized_problem():
    from flashrnn_amd import _lib

    lib = _lib.load()
    # 64 groups x D 1024 x 16 rows x 4 bytes x 2 parities = 8 MiB of exchange alone
    d = _desc(_lib, "elman", 16 * 64, 4, 1, 1024)
    assert lib.frnn_workspace_bytes(ctypes.byref(d), 0) > (8 << 20)
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    rc = lib.frnn_fwd_noalloc(ctypes.byref(d), *([1] * 7), status.data_ptr(), None)
    assert rc == _lib.FRNN_E_SCRATCH
    assert "8 MiB" in _lib.strerror(rc)

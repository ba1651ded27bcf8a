"""GPU tests of the prepared, forward-only path (FlashRNN2's PreparedSequence,
flashrnn/flashrnn2/prepared.py:18-192): output policies full / hidden / last, FP32
snapshots, chunked step windows and HIP-graph replay.

The reference's own check of this path (tools/dispatch_check.py:148-160) is
bitwise agreement with the unchunked, uncaptured run; here:
  * full / BF16 snapshot == flashrnn() states bitwise, final == its FP32 carry;
  * the FP32 snapshot rounded to BF16 == the BF16 snapshot bitwise, and the
    FP32 snapshot against the oracle within the north-star tolerance (1e-2 for
    BF16 operands vs numerics="fp32_state_bf16_mma", 1e-4 FP32 vs "mathematical");
  * hidden == full[0], last == full[0][:, -1:] bitwise;
  * chunked == unchunked and graph replay == eager, bitwise.
"""

import pytest
import torch

from oracle.torch_restatement import flashrnn_torch
from tests.test_gpu_parity import TOL, make, rel

pytestmark = pytest.mark.gpu


def inputs(cell, B, T, N, D, seed, io=torch.bfloat16, zero_state=False):
    cpu, _, _ = make(cell, B, T, N, D, seed, zero_state)
    wx, R, b, s0 = (t.to(io) for t in cpu)
    return [t.cuda().contiguous() for t in (wx, R, b)] + [cpu[3].float().cuda()]


def prepared(args, cell, **kw):
    from flashrnn_amd.prepared import PreparedSequence

    p = PreparedSequence(*args, cell, **kw)
    out, final = p.run()
    p.check()
    return p, out.clone(), final.clone()


CELLS = [("lstm", 5, 24, 2, 64), ("gru", 3, 20, 2, 96), ("elman", 7, 18, 3, 32), ("slstm", 4, 22, 2, 128)]
IDS = [f"{c[0]}-B{c[1]}T{c[2]}N{c[3]}D{c[4]}" for c in CELLS]


@pytest.mark.parametrize("cell,B,T,N,D", CELLS, ids=IDS)
def test_full_matches_flashrnn(cell, B, T, N, D):
    from flashrnn_amd import flashrnn, set_strict

    set_strict(True)
    print(f"\n[prepared] full vs flashrnn {cell} B{B} T{T} N{N} D{D}", flush=True)
    args = inputs(cell, B, T, N, D, seed=21)
    _, out, final = prepared(args, cell)
    with torch.no_grad():
        hist, last = flashrnn(*args, function=cell, dtype="bfloat16")
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and torch.equal(out, hist)
    assert final.dtype == torch.float32 and torch.equal(final, last)


@pytest.mark.parametrize("cell,B,T,N,D", CELLS, ids=IDS)
def test_policies_and_snapshot(cell, B, T, N, D):
    print(f"\n[prepared] policies {cell} B{B} T{T} N{N} D{D}", flush=True)
    args = inputs(cell, B, T, N, D, seed=22)
    _, full, final = prepared(args, cell)
    _, full32, final32 = prepared(args, cell, snapshot_dtype=torch.float32)
    assert full32.dtype == torch.float32 and torch.equal(full32.to(torch.bfloat16), full)
    assert torch.equal(final32, final)
    for mode, expect in (("hidden", full[0]), ("last", full[0][:, -1:])):
        for snap, exp in ((None, expect), (torch.float32, full32[0] if mode == "hidden" else full32[0][:, -1:])):
            _, out, fin = prepared(args, cell, output_mode=mode, snapshot_dtype=snap)
            assert out.shape == exp.shape and torch.equal(out, exp), (mode, snap)
            assert torch.equal(fin, final)
    # the FP32 snapshot against the oracle (inputs as the kernel saw them)
    cpu = [t.float().cpu() for t in args]
    eh, el = flashrnn_torch(*cpu, cell=cell, numerics="fp32_state_bf16_mma")
    assert rel(full32, eh) <= TOL["bfloat16"] and rel(final32, el) <= TOL["bfloat16"]


@pytest.mark.parametrize("cell", ["lstm", "slstm"])
def test_fp32_inputs_vs_oracle(cell):
    print(f"\n[prepared] fp32 {cell} B6 T16 N2 D64", flush=True)
    args = inputs(cell, 6, 16, 2, 64, seed=23, io=torch.float32)
    _, out, final = prepared(args, cell, output_mode="hidden", chunks=[5, 11])
    eh, el = flashrnn_torch(*[t.cpu() for t in args], cell=cell, numerics="mathematical")
    assert rel(out, eh[0]) <= TOL["float32"] and rel(final, el) <= TOL["float32"]


@pytest.mark.parametrize("mode", ["full", "hidden", "last"])
@pytest.mark.parametrize("cell,B,T,N,D", CELLS, ids=IDS)
def test_chunks_equal_unchunked(cell, B, T, N, D, mode):
    print(f"\n[prepared] chunks {mode} {cell} B{B} T{T} N{N} D{D}", flush=True)
    # sLSTM from a zero state: the zero-normalizer predicate belongs to the first window only
    args = inputs(cell, B, T, N, D, seed=24, zero_state=(cell == "slstm"))
    _, out, final = prepared(args, cell, output_mode=mode)
    for chunks in ([1] * 3 + [T - 3], [T // 3, T // 3, T - 2 * (T // 3)], [T - 1, 1]):
        _, co, cf = prepared(args, cell, output_mode=mode, chunks=chunks)
        assert torch.equal(co, out) and torch.equal(cf, final), chunks


def test_graph_replay_tracks_input_updates():
    """Captured once, replayed with the inputs refreshed in place between replays
    (eager work and synchronisation in between); every replay equals a fresh eager run."""
    print("\n[prepared] graph replay lstm B8 T40 N3 D256 hidden chunks [16,24]", flush=True)
    args = inputs("lstm", 8, 40, 3, 256, seed=25)
    from flashrnn_amd.prepared import PreparedSequence

    p = PreparedSequence(*args, "lstm", output_mode="hidden", chunks=[16, 24]).capture()
    g = torch.Generator(device="cuda").manual_seed(5)
    try:
        for rep in range(4):
            if rep:
                args[0].copy_(torch.randn(args[0].shape, generator=g, device="cuda").to(args[0].dtype))
                args[3].copy_(0.5 * torch.randn(args[3].shape, generator=g, device="cuda"))
            torch.cuda.synchronize()
            out, final = p.run()
            got = (out.clone(), final.clone())
            torch.cuda.synchronize()
            _, eo, ef = prepared(args, "lstm", output_mode="hidden")
            assert torch.equal(got[0], eo) and torch.equal(got[1], ef), rep
        p.check()
    finally:
        p.close()


@pytest.mark.parametrize("cell,B,T,N,D", [("lstm", 5, 12, 2, 48), ("slstm", 3, 9, 1, 16), ("gru", 9, 10, 3, 80)],
                         ids=["lstm-D48", "slstm-D16", "gru-D80"])
def test_padded_width(cell, B, T, N, D):
    """Widths that are a multiple of 16 but not of 32 run on padded copies:
    bitwise flashrnn() (which pads the same way), in every policy, in chunks,
    and under graph replay with the caller's tensors updated in place."""
    from flashrnn_amd import flashrnn, set_strict
    from flashrnn_amd.prepared import PreparedSequence

    set_strict(True)
    print(f"\n[prepared] padded width {cell} B{B} T{T} N{N} D{D}", flush=True)
    args = inputs(cell, B, T, N, D, seed=28)
    _, out, final = prepared(args, cell)
    with torch.no_grad():
        hist, last = flashrnn(*args, function=cell, dtype="bfloat16")
    torch.cuda.synchronize()
    assert out.shape == hist.shape and torch.equal(out, hist)
    assert final.shape == last.shape and torch.equal(final, last)
    _, ho, hf = prepared(args, cell, output_mode="hidden", chunks=[T // 2, T - T // 2])
    assert torch.equal(ho, hist[0]) and torch.equal(hf, last)
    _, lo, _ = prepared(args, cell, output_mode="last", snapshot_dtype=torch.float32)
    assert lo.shape == (B, 1, N, D)
    p = PreparedSequence(*args, cell, output_mode="full", chunks=[1, T - 1]).capture()
    g = torch.Generator(device="cuda").manual_seed(6)
    try:
        for rep in range(3):
            if rep:
                args[0].copy_(torch.randn(args[0].shape, generator=g, device="cuda").to(args[0].dtype))
                args[1].copy_((torch.randn(args[1].shape, generator=g, device="cuda") / D**0.5).to(args[1].dtype))
            torch.cuda.synchronize()
            o, f = p.run()
            got = (o.clone(), f.clone())
            torch.cuda.synchronize()
            with torch.no_grad():
                eo, ef = flashrnn(*args, function=cell, dtype="bfloat16")
            torch.cuda.synchronize()
            assert torch.equal(got[0], eo) and torch.equal(got[1], ef), rep
        p.check()
    finally:
        p.close()


def test_headline_head_shape_wide_and_bf16_initial():
    """The C2 head shape with a BF16 initial state (refreshed FP32 copy), and a two-tile (D = 768) head."""
    print("\n[prepared] lstm B8 T64 N3 D256 bf16 initial; gru B16 T12 N1 D768", flush=True)
    args = inputs("lstm", 8, 64, 3, 256, seed=26)
    args[3] = args[3].to(torch.bfloat16)
    _, out, final = prepared(args, "lstm", output_mode="last", chunks=[32, 32])
    cpu = [t.float().cpu() for t in args]
    eh, el = flashrnn_torch(*cpu, cell="lstm", numerics="fp32_state_bf16_mma")
    assert rel(out, eh[0][:, -1:]) <= TOL["bfloat16"] and rel(final, el) <= TOL["bfloat16"]
    args = inputs("gru", 16, 12, 1, 768, seed=27)
    _, out, final = prepared(args, "gru", snapshot_dtype=torch.float32, chunks=[7, 5])
    eh, el = flashrnn_torch(*[t.float().cpu() for t in args], cell="gru", numerics="fp32_state_bf16_mma")
    assert rel(out, eh) <= TOL["bfloat16"] and rel(final, el) <= TOL["bfloat16"]


def test_check_reports_exchange_timeout():
    """A never-ready exchange (forced from the host, spin limit 1): check() raises; a new instance works."""
    import sys

    from flashrnn_amd import _lib
    from flashrnn_amd.prepared import PreparedSequence

    F = sys.modules["flashrnn_amd.flashrnn"]
    print("\n[prepared] timeout lstm B4 T16 N2 D128", flush=True)
    args = inputs("lstm", 4, 16, 2, 128, seed=28)
    lib = _lib.load()
    lib.frnn_set_spin_limit(1)
    F._state["test_unready"] = True
    try:
        p = PreparedSequence(*args, "lstm", output_mode="hidden")
        p.run()
        with pytest.raises(RuntimeError, match="did not arrive|timeout|exchange"):
            p.check()
    finally:
        F._state["test_unready"] = False
        lib.frnn_set_spin_limit(0)
    _, out, _ = prepared(args, "lstm", output_mode="hidden")
    _, full, _ = prepared(args, "lstm")
    assert torch.equal(out, full[0])

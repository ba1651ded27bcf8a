"""Argument checks of the differentiable output-policy call (CPU only; no kernel runs),
after the reference's checks (flashrnn/flashrnn2/training.py:214-228)."""

from types import SimpleNamespace

import pytest
import torch

from flashrnn_amd.training import recurrence


def args(B=2, T=5, N=1, D=64):
    return (torch.zeros(B, T, 4, N, D), torch.zeros(4, N, D, D), torch.zeros(4, N, D), torch.zeros(2, B, 1, N, D))


@pytest.mark.parametrize("kw,match", [
    (dict(output_mode="states"), "output mode"),
    (dict(snapshot_dtype=torch.float16), "snapshot"),
    (dict(sequence_context=SimpleNamespace(step_offset=3)), "continuation"),
    (dict(backward_options={"fast": True}), "backward_options"),
])
def test_option_errors(kw, match):
    with pytest.raises(ValueError, match=match):
        recurrence(*args(), "lstm", **kw)


def test_shape_and_device_errors():
    wx, R, b, s0 = args()
    with pytest.raises(ValueError, match="gates"):
        recurrence(wx[:, :, :3], R, b, s0, "lstm")
    with pytest.raises(ValueError, match="recurrent"):
        recurrence(wx, R[:, :, :3], b, s0, "lstm")
    with pytest.raises(ValueError, match="initial"):
        recurrence(wx, R, b, s0[:1], "lstm")
    with pytest.raises(ValueError, match="cell"):
        recurrence(wx, R, b, s0, "rnn")
    with pytest.raises(ValueError, match="GPU"):
        recurrence(wx, R, b, s0, "lstm")

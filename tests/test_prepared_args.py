"""Argument checks of the prepared path (CPU only; no kernel runs).

They follow the reference's PreparedSequence checks (flashrnn/flashrnn2/prepared.py:18-66),
which raise ValueError before anything is allocated."""

import pytest
import torch

from flashrnn_amd.prepared import KernelConfig, PreparedSequence


def args(cell="lstm", B=2, T=5, N=1, D=64, gw=4, gr=4, gt=4, S=2):
    return (torch.zeros(B, T, gw, N, D), torch.zeros(gr, N, D, D), torch.zeros(gt, N, D), torch.zeros(S, B, 1, N, D))


@pytest.mark.parametrize("kw,match", [
    (dict(output_mode="states"), "output mode"),
    (dict(chunks=[2, 2]), "chunk"),
    (dict(chunks=[5, 0]), "chunk"),
    (dict(chunks=[2.5, 2.5]), "chunk"),
    (dict(snapshot_dtype=torch.float16), "snapshot"),
])
def test_option_errors(kw, match):
    with pytest.raises(ValueError, match=match):
        PreparedSequence(*args(), "lstm", **kw)


def test_shape_errors():
    wx, R, b, s0 = args()
    with pytest.raises(ValueError, match="gates"):
        PreparedSequence(wx[:, :, :3], R, b, s0, "lstm")
    with pytest.raises(ValueError, match="multiple of 16"):
        PreparedSequence(*args(D=40), "lstm")
    with pytest.raises(ValueError, match="multiple of 16"):
        PreparedSequence(*args(D=8), "lstm")
    with pytest.raises(ValueError, match="recurrent"):
        PreparedSequence(wx, R[:3], b, s0, "lstm")
    with pytest.raises(ValueError, match="initial"):
        PreparedSequence(wx, R, b, s0[:1], "lstm")
    with pytest.raises(ValueError, match="cell"):
        PreparedSequence(wx, R, b, s0, "rnn")
    # every check above passed for these: only the device is wrong
    with pytest.raises(ValueError, match="GPU"):
        PreparedSequence(*args("gru", gw=3, gr=3, S=1), "gru")


def test_config():
    with pytest.raises(ValueError, match="exchange"):
        KernelConfig(exchange="nvlink")
    assert KernelConfig().exchange is None

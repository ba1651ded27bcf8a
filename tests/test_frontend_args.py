"""Front-end argument handling of flashrnn() that needs no GPU."""

import pytest
import torch

from flashrnn_amd.flashrnn import io_dtype


def test_io_dtype_same():
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        assert io_dtype(dt, dt, dt) == dt


@pytest.mark.parametrize(
    "wx,r,b",
    [
        (torch.bfloat16, torch.float32, torch.bfloat16),
        (torch.bfloat16, torch.bfloat16, torch.float32),
        (torch.float32, torch.bfloat16, torch.bfloat16),
        (torch.bfloat16, torch.float16, torch.bfloat16),
    ],
)
def test_io_dtype_mixed_promotes_to_fp32(wx, r, b):
    """A mix never rounds an input to a narrower type before the kernel sees it."""
    assert io_dtype(wx, r, b) == torch.float32


def test_io_dtype_rejects_unsupported():
    with pytest.raises(ValueError, match="R dtype"):
        io_dtype(torch.float32, torch.float64, torch.float32)

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


def test_reference_config_fields():
    """Every public field of the reference's FlashRNNConfig constructs here
    (flashrnn/flashrnn/flashrnn.py:121-201); layouts and values are validated."""
    from flashrnn_amd import FlashRNNConfig

    c = FlashRNNConfig(function="gru", backend="cuda_fused", dtype="bfloat16", constants={}, simple_agg=True,
                       hidden_dim=768, num_heads=3, head_dim=256, batch_size=8, input_shape="TBGHD",
                       output_shape="STBHD", recurrent_shape="HPGD", bias_shape="HGD", dtype_acc="float32",
                       dtype_b="float32", dtype_r="bfloat16", dtype_w="bfloat16", dtype_g=None, dtype_s=None,
                       dtype_a=None, enable_automatic_mixed_precision=True, trainable_r=True, trainable_b=[True],
                       initial_val=0.5, forward_clipval=None)
    assert c.simple_agg is False and c.constants == {} and c.num_states == 1
    for kw in (dict(input_shape="BTHGD"), dict(output_shape="SBTHX"), dict(recurrent_shape="GHD"),
               dict(bias_shape="GHDP"), dict(constants={"a": 1.0}), dict(dtype_acc="bfloat16"),
               dict(initial_val=[0.0, 1.0, 2.0])):
        with pytest.raises(ValueError):
            FlashRNNConfig(function="lstm", **kw)
    FlashRNNConfig(function="slstm", initial_val=[0.0, 0.0, 1.0, 0.0])

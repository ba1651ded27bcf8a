"""The projection + recurrence layer: its oracle pinned against torch.nn (CPU), and
the argument checks of flashrnn_amd.layer (CPU, no kernel runs).

``oracle.torch_restatement.flashrnn_layer`` composes the projection with the
pinned ``flashrnn_torch`` restatement; what it adds -- the orientation of the
projection weight -- is pinned by the reference's own layer mapping onto
``torch.nn.LSTM/GRU/RNN`` (``flashrnn/flashrnn2/torch_layer.py:33-57``: per head,
``weight_ih = input_weight[:, head].reshape(G*D, I)``, ``weight_hh`` from R with
GRU's recurrent gate order (1, 2, 0), the bias mapping).
"""

import pytest
import torch

from oracle.torch_restatement import SIZES, flashrnn_layer


def torch_layer_reference(inputs, W, R, b, initial, cell):
    """torch.nn modules under the mapping of torch_layer.py:33-57, one per head."""
    G, N, D, I = W.shape
    hist, finals = [], []
    for n in range(N):
        kind = {"lstm": torch.nn.LSTM, "gru": torch.nn.GRU, "elman": torch.nn.RNN}[cell]
        m = kind(I, D, batch_first=True, dtype=torch.float64)
        with torch.no_grad():
            m.weight_ih_l0.copy_(W[:, n].reshape(G * D, I))
            m.weight_hh_l0.copy_(R[[1, 2, 0] if cell == "gru" else list(range(G)), n].reshape(G * D, D))
            m.bias_hh_l0.zero_()
            if cell == "gru":
                m.bias_ih_l0.copy_(b[[1, 2, 3], n].reshape(-1))
                m.bias_hh_l0[2 * D:].copy_(b[0, n])
            else:
                m.bias_ih_l0.copy_(b[:, n].reshape(-1))
        h0 = initial[0, :, 0, n].unsqueeze(0).contiguous()
        if cell == "lstm":
            out, (hT, cT) = m(inputs, (h0, initial[1, :, 0, n].unsqueeze(0).contiguous()))
            finals.append(torch.stack((hT[0], cT[0])))
        else:
            out, hT = m(inputs, h0)
            finals.append(hT)
        hist.append(out)
    return torch.stack(hist, dim=2), torch.stack(finals, dim=2).unsqueeze(2)


@pytest.mark.parametrize("cell", ["lstm", "gru", "elman"])
def test_layer_oracle_is_torch_nn(cell):
    g = torch.Generator().manual_seed(61)
    G, T_, S = SIZES[cell][0], 7, SIZES[cell][2]
    B, N, D, I = 3, 2, 4, 5
    Gr = {"lstm": 4, "gru": 3, "elman": 1}[cell]
    x = torch.randn(B, T_, I, generator=g, dtype=torch.float64)
    W = torch.randn(G, N, D, I, generator=g, dtype=torch.float64) / I**0.5
    R = torch.randn(Gr, N, D, D, generator=g, dtype=torch.float64) / D**0.5
    b = 0.1 * torch.randn(SIZES[cell][1], N, D, generator=g, dtype=torch.float64)
    s0 = torch.randn(S, B, 1, N, D, generator=g, dtype=torch.float64)
    h, last = flashrnn_layer(x, W, R, b, s0, cell=cell)
    eh, elast = torch_layer_reference(x, W, R, b, s0, cell)
    torch.testing.assert_close(h, eh, atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(last, elast, atol=1e-12, rtol=1e-12)


def _layer_args(cell="lstm", B=2, T=5, N=1, D=64, I=48):
    gr, gw, gt, S = {"lstm": (4, 4, 4, 2), "gru": (3, 3, 4, 1), "elman": (1, 1, 1, 1), "slstm": (4, 4, 4, 4)}[cell]
    return (torch.zeros(B, T, I), torch.zeros(gw, N, D, I), torch.zeros(gr, N, D, D), torch.zeros(gt, N, D),
            torch.zeros(S, B, 1, N, D))


def test_layer_argument_errors():
    from flashrnn_amd.layer import FlashRNNLayer, flashrnn_projected

    x, W, R, b, s0 = _layer_args()
    with pytest.raises(ValueError, match="input weight"):
        flashrnn_projected(x, W[:3], R, b, s0, "lstm")
    with pytest.raises(ValueError, match="inputs"):
        flashrnn_projected(x[:, :, :7], W, R, b, s0, "lstm")
    with pytest.raises(ValueError, match="recurrent"):
        flashrnn_projected(x, W, R[:2], b, s0, "lstm")
    with pytest.raises(ValueError, match="initial"):
        flashrnn_projected(x, W, R, b, s0[:1], "lstm")
    with pytest.raises(ValueError, match="GPU"):
        flashrnn_projected(x, W, R, b, s0, "lstm")
    with pytest.raises(ValueError, match="bias"):
        FlashRNNLayer(W, R, b[:2], "lstm")
    with pytest.raises(ValueError, match="dtype"):
        FlashRNNLayer(W, R, b, "lstm", dtype="float64")
    layer = FlashRNNLayer(W, R, b, "lstm")
    assert sorted(n for n, _ in layer.named_parameters()) == ["bias", "input_weight", "recurrent"]

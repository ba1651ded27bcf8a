"""Write the BASELINE config-1 fixture (LSTM, FP32 inputs, forward, B4 T64 N1 D64).

The expected outputs come from ``torch.nn.LSTM`` in FP64 -- a textbook
library routine, not the reference's code -- under the gate mapping of the
reference's own layer (``flashrnn/flashrnn2/torch_layer.py:33-57``: gate
order i, f, z(g), o; ``weight_hh = R.reshape(4D, D)`` with R acting on the
left; identity input weights, so the LSTM's input is Wx itself; the bias in
``bias_ih``). The reference equates its ``flashrnn_torch`` with that module to
1e-12 (``tests/flashrnn2/test_torch_layer.py``), so the fixture pins the
oracle and the FP32 kernel without importing the reference.

Inputs follow config 1: Wx ~ N(0,1), R ~ N(0,1/D), b ~ N(0, 0.1^2),
initial states ~ N(0,1), seed 20261001, drawn in FP32 (the fixture stores the
FP32 inputs; the FP64 module sees exactly those values).

Usage: ``python tests/golden/make_c1.py`` (writes ``c1_lstm_fp32.npz`` here).
"""

from __future__ import annotations

import pathlib

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent
B, T, N, D, SEED = 4, 64, 1, 64, 20261001


def inputs():
    g = torch.Generator().manual_seed(SEED)
    wx = torch.randn(B, T, 4, N, D, generator=g)
    R = torch.randn(4, N, D, D, generator=g) / D**0.5
    b = 0.1 * torch.randn(4, N, D, generator=g)
    s0 = torch.randn(2, B, 1, N, D, generator=g)
    return wx, R, b, s0


def library_forward(wx, R, b, s0):
    """hist [2,B,T,N,D] and last [2,B,1,N,D] from torch.nn.LSTM in FP64, head by head."""
    hist = torch.empty(2, B, T, N, D, dtype=torch.float64)
    last = torch.empty(2, B, 1, N, D, dtype=torch.float64)
    for n in range(N):
        m = torch.nn.LSTM(4 * D, D, batch_first=True, dtype=torch.float64)
        with torch.no_grad():
            m.weight_ih_l0.copy_(torch.eye(4 * D, dtype=torch.float64))
            m.weight_hh_l0.copy_(R[:, n].double().reshape(4 * D, D))
            m.bias_ih_l0.copy_(b[:, n].double().reshape(-1))
            m.bias_hh_l0.zero_()
            x = wx[:, :, :, n].double().reshape(B, T, 4 * D)
            h0 = s0[0, :, 0, n].double()[None]
            c0 = s0[1, :, 0, n].double()[None]
            out, (hT, cT) = m(x, (h0, c0))
            # torch.nn.LSTM returns the hidden history only; the cell history is
            # rebuilt by running one step at a time from the same module
            cs, hc = [], (h0, c0)
            for t in range(T):
                _, hc = m(x[:, t : t + 1], hc)
                cs.append(hc[1][0])
        hist[0, :, :, n] = out
        hist[1, :, :, n] = torch.stack(cs, 1)
        last[0, :, 0, n] = hT[0]
        last[1, :, 0, n] = cT[0]
    return hist, last


def main():
    wx, R, b, s0 = inputs()
    hist, last = library_forward(wx, R, b, s0)
    np.savez_compressed(
        HERE / "c1_lstm_fp32.npz",
        wx=wx.numpy(), R=R.numpy(), b=b.numpy(), s0=s0.numpy(),
        hist=hist.numpy(), last=last.numpy(),
    )
    print("wrote c1_lstm_fp32.npz")


if __name__ == "__main__":
    main()

"""flashrnn_amd: MI355X-native (gfx950) fused recurrent forward/backward.

Drop-in for the fused backend of FlashRNN's ``flashrnn()``
(``flashrnn/flashrnn/flashrnn.py:1117-1138``): LSTM, GRU, Elman and sLSTM
cells with the public ``[S,B,T,N,D]`` state layout, implemented by
hand-written HIP kernels behind the C ABI of ``include/frnn.h``.
"""

from .flashrnn import FlashRNNConfig, flashrnn, set_strict, synchronize_and_check

__all__ = ["flashrnn", "FlashRNNConfig", "set_strict", "synchronize_and_check"]

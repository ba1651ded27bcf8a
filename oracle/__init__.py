"""CPU oracle for the fused recurrent forward/backward path.

TEST INFRASTRUCTURE ONLY. Nothing in the product (``flashrnn_amd``) imports,
links or calls anything in this package. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use it,
and only as the checker or as the timed CPU baseline.

Contents:

* ``torch_restatement`` -- a restatement, in CPU PyTorch ops, of the
  reference's ``flashrnn_torch`` oracle
  (``flashrnn/flashrnn2/torch_backend.py:12-67``) and its per-step
  ``recurrence`` (``flashrnn/flashrnn2/reference.py:24-114``). Backward is
  torch autograd, as in the reference.
* ``numpy_explicit`` -- an independent NumPy restatement of the same forward
  with a hand-derived backward, including the BF16 operand/cotangent rounding
  of the ``fp32_state_bf16_mma`` policy. It pins the autograd restatement
  (and documents the backward the HIP kernels implement).

Pinning (see ``tests/test_oracle.py``): library known answers (``torch.nn``
LSTM/GRU/RNN for the mathematical LSTM/GRU/Elman cells), closed forms (Elman
with R=0, sLSTM normalizer known answer ``m = 2 - log 2``, zero-state single
steps), invariants (chunked == unchunked bitwise, gradcheck, BF16 policy ==
step-by-step restatement bitwise), the explicit-backward cross-check, and
golden vectors written by the real reference (``tests/golden``).
"""

"""CPU restatement of greedy token selection (test infrastructure only).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg, never by the product package.

The reference selects greedy tokens with ``logits.argmax(-1)``
(microinfer/runner.py:236-240, captured into each decode graph; :618-625;
microinfer/layer/sampler.py:44-45). torch's argmax orders values by ">"
with NaN above every number, and returns the first index among equal maxima
(so +0 and -0 tie, and a row of -inf selects index 0).

Pins (tests/test_oracle_greedy.py): torch.argmax on the CPU and a
pure-Python scan on rows built around each special case (ties, NaN
anywhere, +/-0, +/-inf, all -inf, one-element rows, subnormals), and
numpy's argmax, which documents the same first-occurrence and NaN rule.
"""

from __future__ import annotations

import numpy as np


def greedy_argmax(logits: np.ndarray) -> np.ndarray:
    """int64 ``[rows]``: per row, the first NaN's index if the row holds a
    NaN, else the first index of the row's maximum (runner.py:240)."""
    x = np.asarray(logits)
    if x.ndim != 2 or x.shape[1] == 0:
        raise ValueError("logits must be [rows, vocab] with vocab > 0")
    x = x.astype(np.float64)  # exact for fp16 / bf16 / fp32 inputs
    nan = np.isnan(x)
    has_nan = nan.any(axis=1)
    finite_max = np.argmax(np.where(nan, -np.inf, x), axis=1)
    return np.where(has_nan, np.argmax(nan, axis=1), finite_max).astype(np.int64)

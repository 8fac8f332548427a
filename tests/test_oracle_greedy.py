"""Pins of the greedy-selection oracle (oracle/greedy.py), CPU only.

torch.argmax on the CPU is the routine the reference calls
(microinfer/runner.py:240); a pure-Python scan that keeps the first strict
maximum and stops at the first NaN is the brute-force statement of the same
order; numpy's argmax documents the same rule. Each special case is a row on
which a plausible slip gives another index: the last instead of the first of
equal maxima, NaN skipped instead of winning, -0 ranked below +0, -inf rows
returning nothing, or a 16-bit row widened wrongly.
"""

import math

import numpy as np
import pytest
import torch

from oracle.greedy import greedy_argmax

NAN, INF = float("nan"), float("inf")


def _scan(row):
    best = 0
    for i, v in enumerate(row):
        if math.isnan(v):
            return i
        if v > row[best]:
            best = i
    return best


SPECIAL_ROWS = [
    [3.0, 1.0, 3.0, 2.0],               # equal maxima: the first
    [1.0, NAN, 5.0, NAN],               # NaN wins, the first NaN
    [NAN, 2.0],
    [-INF, -INF, -INF],                 # all -inf: index 0
    [-0.0, 0.0, -0.0],                  # +0 and -0 tie
    [0.0, -0.0],
    [-1.0, -0.5, -2.0],
    [1.0, INF, INF, 2.0],
    [7.0],
    [1e-45, 2e-45, 0.0, -1e-45],        # float32 subnormals
    [-5.0, -INF, -4.0, -4.0],
]


@pytest.mark.parametrize("row", SPECIAL_ROWS, ids=range(len(SPECIAL_ROWS)))
def test_special_rows_match_torch_scan_and_numpy(row):
    x = np.array([row], dtype=np.float32)
    got = int(greedy_argmax(x)[0])
    assert got == int(torch.argmax(torch.from_numpy(x), dim=-1)[0])
    assert got == _scan([float(v) for v in x[0]])
    assert got == int(np.argmax(x[0]))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_random_rows_with_ties_match_torch(dtype):
    gen = torch.Generator().manual_seed(0)
    # Few distinct values, so rows hold many equal maxima; a NaN in some rows.
    x = torch.randint(-4, 5, (64, 1000), generator=gen).to(dtype)
    x[5, 17] = NAN
    x[9, 999] = NAN
    x[9, 3] = NAN
    x[12] = -INF
    want = torch.argmax(x, dim=-1).numpy()
    got = greedy_argmax(x.float().numpy())
    np.testing.assert_array_equal(got, want)
    assert got[5] == 17 and got[9] == 3 and got[12] == 0
    for r in (0, 1, 63):
        assert got[r] == _scan(x[r].float().tolist())


def test_wide_rows_match_torch_and_scan():
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(4, 151936, generator=gen).to(torch.bfloat16)
    x[2, 100000] = x[2].max()  # a later copy of the maximum does not win
    want = torch.argmax(x, dim=-1).numpy()
    got = greedy_argmax(x.float().numpy())
    np.testing.assert_array_equal(got, want)
    assert got[3] == _scan(x[3].float().tolist())


def test_rejects_empty_vocab_and_wrong_rank():
    with pytest.raises(ValueError):
        greedy_argmax(np.zeros((2, 0), dtype=np.float32))
    with pytest.raises(ValueError):
        greedy_argmax(np.zeros(5, dtype=np.float32))

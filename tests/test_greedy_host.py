"""Host side of greedy token selection (no GPU).

CPU tensors raise RuntimeError (the product has no CPU fallback); the C entry
rejects bad sizes, pointers and state with a status and a message before
launching anything.
"""

import pytest
import torch

from microinfer_amd import _lib
from microinfer_amd.layer.hip_sampler import greedy_argmax


def test_cpu_tensors_raise_runtime_error():
    with pytest.raises(RuntimeError, match="HIP device only"):
        greedy_argmax(torch.zeros(2, 8))


def _call(lib, **over):
    args = dict(logits=1024, stride=1000, rows=4, vocab=1000, dtype=2, tokens=4096, state=8192,
                state_bytes=512)
    args.update(over)
    return lib.mi_greedy_argmax(*args.values(), None)


def test_c_entry_validates_before_launch():
    lib = _lib.load()
    assert lib.mi_greedy_argmax_state_bytes(4) == 512  # one 128-byte line per row
    assert lib.mi_greedy_argmax_state_bytes(0) == 0
    assert _call(lib, dtype=7) == 1 and "dtype" in _lib.last_error()
    assert _call(lib, vocab=0) == 1 and _call(lib, rows=-1) == 1
    assert _call(lib, vocab=(1 << 30) + 1, stride=1 << 31) == 2
    assert _call(lib, logits=None) == 1 and "null" in _lib.last_error()
    assert _call(lib, tokens=None) == 1
    assert _call(lib, stride=999) == 1 and "row_stride" in _lib.last_error()
    assert _call(lib, logits=1025) == 1 and "misaligned" in _lib.last_error()
    assert _call(lib, tokens=4100) == 1
    assert _call(lib, state=None) == 3 and "state" in _lib.last_error()
    assert _call(lib, state_bytes=511) == 3
    assert _call(lib, state=8196) == 3
    assert _call(lib, rows=0) == 0  # nothing to do
    assert _lib.last_error() == ""


def test_sampler_validation_matches_the_reference_contract():
    # microinfer/layer/sampler.py:10-31: shape, temperature and logits checks
    # run before any device work.
    from microinfer_amd.layer.hip_sampler import Sampler

    sampler = Sampler()
    good = torch.zeros(2, 5)
    temps = torch.ones(2)
    with pytest.raises(ValueError, match="floating"):
        sampler.probabilities(torch.zeros(2, 5, dtype=torch.int64), temps)
    with pytest.raises(ValueError, match="temperature shape"):
        sampler.probabilities(good, torch.ones(3))
    with pytest.raises(ValueError, match="finite and positive"):
        sampler.probabilities(good, torch.tensor([1.0, 0.0]))
    with pytest.raises(ValueError, match="NaN"):
        sampler.probabilities(torch.tensor([[0.0, float("nan")], [0.0, 1.0]]), temps)
    with pytest.raises(ValueError, match="finite values"):
        sampler.probabilities(torch.full((2, 3), float("-inf")), temps)
    p = sampler.probabilities(torch.tensor([[0.0, 1.0, 2.0], [5.0, 5.0, 5.0]]),
                              torch.tensor([1.0, 0.5]))
    torch.testing.assert_close(p.sum(-1), torch.ones(2))
    torch.testing.assert_close(p[1], torch.full((3,), 1 / 3))
    assert p[0].argmax() == 2

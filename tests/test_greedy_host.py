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

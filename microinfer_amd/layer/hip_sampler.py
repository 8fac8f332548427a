"""Greedy token selection through the HIP library.

``greedy_argmax(logits)`` is ``logits.argmax(-1)`` for ``[rows, vocab]``
logits: what ``ModelRunner._capture_bucket`` records into every decode graph
(microinfer/runner.py:236-240) and what ``ModelRunner.run`` and
``Sampler.sample(greedy=True)`` call for greedy rows (runner.py:618-625,
microinfer/layer/sampler.py:44-45). Same order as torch: NaN above every
number, the first index among equal maxima. One launch, no allocation in the
steady state and no memset, so it can sit inside a captured decode graph.
"""

from __future__ import annotations

import torch

from microinfer_amd import _lib

_FLOAT_DTYPES = (torch.float16, torch.bfloat16, torch.float32)

# Row slots and arrival counters: one zero-filled array per (device, stream),
# left zero by every launch. It is created on a stream's first call, so code
# that captures a graph calls once on the capture stream beforehand (as
# DecodeGraphRunner's warm-up does) to keep the allocation and its zero fill
# out of the graph. An array outgrown by a larger batch stays alive: a
# captured graph may still point at it.
_states: dict[tuple[int, int], torch.Tensor] = {}
_retired_states: list[torch.Tensor] = []


def _state(device: torch.device, stream: int, rows: int) -> torch.Tensor:
    key = (device.index, stream)
    words = _lib.load().mi_greedy_argmax_state_bytes(rows) // 8
    state = _states.get(key)
    if state is None or state.numel() < words:
        if state is not None:
            _retired_states.append(state)
        state = torch.zeros(max(words, 16 * 64), dtype=torch.int64, device=device)
        _states[key] = state
    return state


def greedy_argmax(logits: torch.Tensor, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """int64 ``[rows]`` index of each row's maximum (``logits.argmax(-1)``).

    ``logits`` is float16, bfloat16 or float32 ``[rows, vocab]`` with
    contiguous rows (any row stride); ``out`` optionally receives the tokens.
    """
    _lib.require_device(logits, out, what="greedy argmax")
    if logits.dtype not in _FLOAT_DTYPES:
        raise ValueError("logits must be float16, bfloat16 or float32")
    if logits.ndim != 2 or logits.shape[1] == 0:
        raise ValueError("logits must be [rows, vocab] with vocab > 0")
    if logits.shape[1] > 2 ** 30:
        raise ValueError("vocab must be at most 2^30")
    if logits.stride(1) != 1 or (logits.shape[0] > 1 and logits.stride(0) < logits.shape[1]):
        logits = logits.contiguous()
    rows = logits.shape[0]
    if out is None:
        out = torch.empty(rows, dtype=torch.int64, device=logits.device)
    elif out.dtype != torch.int64 or out.shape != (rows,) or not out.is_contiguous():
        raise ValueError("out must be a contiguous int64 [rows] tensor")
    if rows == 0:
        return out
    stream = _lib.stream_handle(logits.device)
    state = _state(logits.device, stream, rows)
    status = _lib.load().mi_greedy_argmax(
        logits.data_ptr(), logits.stride(0), rows, logits.shape[1], _lib.dtype_code(logits.dtype),
        out.data_ptr(), state.data_ptr(), state.numel() * 8, stream)
    _lib.check(status, "mi_greedy_argmax")
    return out


class Sampler:
    """Temperature sampling with the device argmax.

    Mirrors ``Sampler`` (microinfer/layer/sampler.py:5-50): probabilities
    are a softmax of the row-centred logits over the temperature; a sample is
    ``argmax(probabilities / noise)`` with exponential noise (the
    Gumbel-max construction), taken with ``greedy_argmax``; ``greedy=True``
    returns the argmax of the logits. ``validate`` checks the same contract.
    """

    def __init__(self, validate: bool = True):
        self.validate = validate

    def _validate(self, logits, temperatures):
        if logits.ndim != 2 or logits.shape[1] == 0 or not logits.dtype.is_floating_point:
            raise ValueError("logits must be floating [requests, vocabulary]")
        if temperatures.shape != (logits.shape[0],) or temperatures.device != logits.device:
            raise ValueError("temperature shape/device does not match logits")
        if not torch.isfinite(temperatures).all() or (temperatures <= 0).any():
            raise ValueError("temperatures must be finite and positive")
        if (torch.isnan(logits).any() or torch.isposinf(logits).any()
                or not torch.isfinite(logits).any(-1).all()):
            raise ValueError("each logits row must contain finite values, without NaN/+inf")

    def probabilities(self, logits, temperatures):
        if self.validate:
            self._validate(logits, temperatures)
        work = logits.float()
        work = (work - work.amax(-1, keepdim=True)) / temperatures[:, None]
        return work.softmax(-1)

    def sample(self, logits, temperatures, *, generator=None, greedy=False):
        probabilities = self.probabilities(logits, temperatures)
        if greedy:
            return greedy_argmax(logits)
        noise = torch.empty_like(probabilities).exponential_(generator=generator)
        return greedy_argmax(probabilities / noise)

    def __call__(self, logits, temperatures):
        return self.sample(logits, temperatures)

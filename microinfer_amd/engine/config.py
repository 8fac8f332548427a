"""Engine limits and per-request sampling values.

Mirrors ``SampleParameter`` (microinfer/config/samplepara.py:5-17) and the
fields of ``EngineConfig`` (microinfer/config/engine.py:6-68) that this
engine acts on, with the same validation errors. The reference's switches
for torch.compile and n-gram speculative decoding have no counterpart here:
decode runs from hipGraphs of the HIP kernels, and speculation is not part
of the attention path.
"""

from __future__ import annotations

import math
from dataclasses import dataclass


@dataclass(slots=True)
class SampleParameter:
    temperature: float = 1.0
    max_tokens: int = 64
    ignore_eos: bool = False
    greedy: bool = False

    def __post_init__(self):
        # A temperature near zero is rejected: greedy decoding is asked for
        # with ``greedy=True`` instead (samplepara.py:12-14).
        assert math.isfinite(self.temperature) and self.temperature > 1e-10, (
            "greedy sampling is not permitted"
        )
        if type(self.max_tokens) is not int or self.max_tokens <= 0:
            raise ValueError("max_tokens must be a positive integer")


@dataclass(frozen=True)
class EngineConfig:
    max_num_seqs: int = 16
    max_num_batched_tokens: int = 512
    max_num_prefill_tokens: int = 512  # cap of one prefill chunk
    max_model_len: int = 4096
    eos_token_id: int | None = None
    debug_mode: bool = False
    use_cuda_graph: bool = False  # decode buckets replayed from hipGraphs
    mixed_batch: bool = True  # fill the budget with prefill after running decode

    def __post_init__(self):
        for name in ("max_num_seqs", "max_num_batched_tokens", "max_num_prefill_tokens",
                     "max_model_len"):
            value = getattr(self, name)
            if type(value) is not int or value <= 0:
                raise ValueError(f"{name} must be a positive integer")
        if self.eos_token_id is not None and (
                type(self.eos_token_id) is not int or self.eos_token_id < 0):
            raise ValueError("eos_token_id must be a nonnegative integer or None")
        for name in ("debug_mode", "use_cuda_graph", "mixed_batch"):
            if type(getattr(self, name)) is not bool:
                raise ValueError(f"{name} must be a boolean")

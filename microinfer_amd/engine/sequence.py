"""A request as the scheduler and the runner see it.

Mirrors ``Sequence`` / ``SequenceStatus`` (microinfer/engine/sequence.py:
8-78): token ids (prompt then completion), the block table, how many tokens
are already in the KV cache and how many the current step schedules. The
class attribute ``block_size`` is set by the scheduler on admission.
"""

from __future__ import annotations

from enum import Enum, auto
from itertools import count

from microinfer_amd.engine.config import SampleParameter


class SequenceStatus(Enum):
    WAITING = auto()
    RUNNING = auto()
    FINISHED = auto()


class Sequence:
    block_size = 256
    counter = count()

    def __init__(self, token_ids: list[int], sampling_params: SampleParameter | None = None):
        params = sampling_params or SampleParameter()
        if not token_ids or any(type(t) is not int or t < 0 for t in token_ids):
            raise ValueError("token_ids must be nonempty nonnegative integers")
        self.seq_id = next(Sequence.counter)
        self.status = SequenceStatus.WAITING
        self.token_ids = list(token_ids)
        self.last_token = self.token_ids[-1]
        self.num_tokens = len(self.token_ids)
        self.num_prompt_tokens = self.num_tokens
        self.num_cached_tokens = 0
        self.num_scheduled_tokens = 0
        self.is_prefill = True
        self.block_table: list[int] = []
        self.temperature = params.temperature
        self.max_tokens = params.max_tokens
        self.ignore_eos = params.ignore_eos
        self.greedy = params.greedy
        self.finish_reason: str | None = None

    def __len__(self):
        return self.num_tokens

    def __getitem__(self, key):
        return self.token_ids[key]

    @property
    def is_finished(self) -> bool:
        return self.status == SequenceStatus.FINISHED

    @property
    def num_completion_tokens(self) -> int:
        return self.num_tokens - self.num_prompt_tokens

    @property
    def prompt_token_ids(self) -> list[int]:
        return self.token_ids[:self.num_prompt_tokens]

    @property
    def completion_token_ids(self) -> list[int]:
        return self.token_ids[self.num_prompt_tokens:]

    @property
    def num_blocks(self) -> int:
        return -(-self.num_tokens // self.block_size)

    @property
    def last_block_num_tokens(self) -> int:
        return self.num_tokens - (self.num_blocks - 1) * self.block_size

    def block(self, i: int) -> list[int]:
        """Token ids of logical block ``i``."""
        assert 0 <= i < self.num_blocks
        start = i * self.block_size
        return self.token_ids[start:start + self.block_size]

    def append_token(self, token_id: int) -> None:
        self.token_ids.append(token_id)
        self.last_token = token_id
        self.num_tokens += 1

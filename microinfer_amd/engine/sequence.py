"""One request's state: its tokens, its cache blocks and its step bookkeeping.

Interface of ``Sequence`` / ``SequenceStatus`` (microinfer/engine/sequence.py:
8-78), which the scheduler, the block manager, the runner and the reference's
tests address by name: ``token_ids``, ``num_tokens``, ``num_prompt_tokens``,
``num_cached_tokens``, ``num_scheduled_tokens``, ``is_prefill``,
``block_table``, ``status``, ``finish_reason``, the sampling values and the
block geometry (``num_blocks``, ``block(i)``, ``last_block_num_tokens``).

Layout here: the token list is the only stored sequence data; its length,
last token and the prompt/completion split are derived from it and from the
prompt length, so they cannot disagree. The sampling values stay in the
request's ``SampleParameter`` and are read through it. Status changes go
through three lifecycle calls (``start_running``, ``requeue``, ``finish``)
that set every field a transition touches.
"""

from __future__ import annotations

from enum import Enum, auto
from itertools import count

from microinfer_amd.engine.config import SampleParameter


class SequenceStatus(Enum):
    WAITING = auto()
    RUNNING = auto()
    FINISHED = auto()


def _checked_tokens(token_ids) -> list[int]:
    tokens = list(token_ids)
    if not tokens:
        raise ValueError("a request needs at least one prompt token")
    for t in tokens:
        if type(t) is not int or t < 0:
            raise ValueError(f"prompt token {t!r} is not a nonnegative int")
    return tokens


class Sequence:
    # Tokens per KV block; the scheduler sets it on admission.
    block_size = 256
    # Request ids, increasing in creation order.
    counter = count()

    def __init__(self, token_ids: list[int], sampling_params: SampleParameter | None = None):
        self._tokens = _checked_tokens(token_ids)
        self._prompt_len = len(self._tokens)
        self.sampling = sampling_params if sampling_params is not None else SampleParameter()
        self.seq_id = next(Sequence.counter)
        self.status = SequenceStatus.WAITING
        self.finish_reason: str | None = None
        self.block_table: list[int] = []
        # Tokens whose K/V rows are in the cache, and tokens the current step
        # computes (zero between steps).
        self.num_cached_tokens = 0
        self.num_scheduled_tokens = 0
        self.is_prefill = True

    # -- tokens -------------------------------------------------------------
    @property
    def token_ids(self) -> list[int]:
        return self._tokens

    @token_ids.setter
    def token_ids(self, tokens: list[int]) -> None:
        # Replacing the list (a rollback to fewer tokens) keeps the prompt
        # split inside it.
        self._tokens = list(tokens)
        self._prompt_len = min(self._prompt_len, len(self._tokens))

    @property
    def num_tokens(self) -> int:
        return len(self._tokens)

    @num_tokens.setter
    def num_tokens(self, n: int) -> None:
        """Truncate to the first ``n`` tokens (a length is never grown this way)."""
        if not 0 < n <= len(self._tokens):
            raise ValueError(f"cannot set the length of a {len(self._tokens)}-token "
                             f"sequence to {n}")
        self.token_ids = self._tokens[:n]

    @property
    def num_prompt_tokens(self) -> int:
        return self._prompt_len

    @property
    def last_token(self) -> int:
        return self._tokens[-1]

    @property
    def num_completion_tokens(self) -> int:
        return len(self._tokens) - self._prompt_len

    @property
    def prompt_token_ids(self) -> list[int]:
        return self._tokens[: self._prompt_len]

    @property
    def completion_token_ids(self) -> list[int]:
        return self._tokens[self._prompt_len:]

    def __len__(self) -> int:
        return len(self._tokens)

    def __getitem__(self, key):
        return self._tokens[key]

    def append_token(self, token_id: int) -> None:
        self._tokens.append(token_id)

    # -- sampling values ----------------------------------------------------
    @property
    def temperature(self) -> float:
        return self.sampling.temperature

    @property
    def max_tokens(self) -> int:
        return self.sampling.max_tokens

    @property
    def ignore_eos(self) -> bool:
        return self.sampling.ignore_eos

    @property
    def greedy(self) -> bool:
        return self.sampling.greedy

    # -- block geometry -----------------------------------------------------
    @property
    def num_blocks(self) -> int:
        full, rest = divmod(len(self._tokens), self.block_size)
        return full + (rest > 0)

    @property
    def last_block_num_tokens(self) -> int:
        rest = len(self._tokens) % self.block_size
        return rest if rest else min(self.block_size, len(self._tokens))

    def block(self, i: int) -> list[int]:
        """Token ids of logical block ``i`` (AssertionError outside the sequence)."""
        if not 0 <= i < self.num_blocks:
            raise AssertionError(f"block {i} outside 0..{self.num_blocks - 1}")
        lo = i * self.block_size
        return self._tokens[lo:lo + self.block_size]

    # -- lifecycle ----------------------------------------------------------
    @property
    def is_finished(self) -> bool:
        return self.status is SequenceStatus.FINISHED

    def start_running(self) -> None:
        """The whole prompt is scheduled: from now on the request decodes."""
        self.status = SequenceStatus.RUNNING

    def requeue(self) -> None:
        """Back to waiting with every token kept, to be prefilled again."""
        self.status = SequenceStatus.WAITING
        self.is_prefill = True
        self.num_scheduled_tokens = 0

    def finish(self, reason: str) -> None:
        self.status = SequenceStatus.FINISHED
        self.finish_reason = reason
        self.num_scheduled_tokens = 0

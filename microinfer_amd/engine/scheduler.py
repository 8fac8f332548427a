"""Step scheduling for the engine: which requests run next, and how many tokens.

Counterpart of ``Scheduler`` (microinfer/engine/scheduler.py:8-260) without
the speculative-decoding hooks. The decisions are the ones the reference's
tests pin (tests/components/test_scheduler.py), restated as rules:

1. A step has a token budget (``max_num_batched_tokens``) and a seat budget
   (``max_num_seqs``).
2. With ``mixed_batch`` the running requests are served first, one decode
   token each, oldest first; the ones served move to the back of the running
   queue, so a budget too small for all of them rotates through them. The
   budget left over then goes to waiting prompts. Without ``mixed_batch``
   prompts go first and decode runs only in a step with no prompt work.
3. Prompts are taken in arrival order. A prompt that has no blocks yet is
   admitted when the block manager can hold it (reusing cached full-block
   prefixes); its chunk is capped by the budget and by
   ``max_num_prefill_tokens``. A chunk that does not finish its prompt is the
   last prompt work of the step. A prompt whose last chunk is scheduled
   becomes a running request.
4. A running request that needs a fresh block when none is free evicts the
   newest running request (which goes back to the front of the waiting queue
   with all its tokens, to be prefilled again); with nobody else left it
   evicts itself.
5. After the step, ``postprocess`` publishes the hashes of completed blocks,
   advances each request's cached count, drops the sample of a prompt chunk
   that did not reach the end of its prompt, and finishes requests on EOS or
   on the length limits.

The implementation is organised around a ``_StepBuilder`` that owns the two
budgets and records the step's entries; the two policies only choose the
order in which its decode and prompt passes run.
"""

from __future__ import annotations

from collections import deque

from microinfer_amd.engine.blockmanager import BlockManager
from microinfer_amd.engine.config import EngineConfig
from microinfer_amd.engine.sequence import Sequence, SequenceStatus


_COUNTERS = ("num_preemptions", "num_steps", "num_prefill_steps", "num_decode_steps",
             "num_mixed_steps")


class _StepBuilder:
    """The entries of one step under a token budget and a seat budget."""

    def __init__(self, tokens: int, seats: int):
        self.tokens = tokens
        self.seats = seats
        self.entries: list[Sequence] = []

    def has_room(self) -> bool:
        return self.tokens > 0 and len(self.entries) < self.seats

    def add(self, seq: Sequence, num_tokens: int, prefill: bool) -> None:
        seq.num_scheduled_tokens = num_tokens
        seq.is_prefill = prefill
        self.tokens -= num_tokens
        self.entries.append(seq)


class Scheduler:
    def __init__(self, config: EngineConfig, block_manager: BlockManager):
        self.config = config
        self.block_manager = block_manager
        self.block_size = block_manager.block_size
        self.max_num_seqs = config.max_num_seqs
        self.max_num_batched_tokens = config.max_num_batched_tokens
        self.eos = config.eos_token_id
        self.waiting: deque[Sequence] = deque()
        self.running: deque[Sequence] = deque()
        # The step handed out by schedule() and not yet postprocessed.
        self._inflight: tuple[list[Sequence], bool] | None = None
        self._counts = dict.fromkeys(_COUNTERS, 0)

    # -- observability (the counters never affect a decision) ------------------
    num_preemptions = property(lambda self: self._counts["num_preemptions"])
    num_steps = property(lambda self: self._counts["num_steps"])
    num_prefill_steps = property(lambda self: self._counts["num_prefill_steps"])
    num_decode_steps = property(lambda self: self._counts["num_decode_steps"])
    num_mixed_steps = property(lambda self: self._counts["num_mixed_steps"])

    def stats(self) -> dict:
        return {"waiting": len(self.waiting), "running": len(self.running), **self._counts}

    @property
    def max_length(self) -> int:
        """Longest a request may grow: the model limit or the whole cache."""
        cache_tokens = len(self.block_manager.blocks) * self.block_size
        return min(self.config.max_model_len, cache_tokens)

    def is_finished(self) -> bool:
        return not (self.waiting or self.running)

    # -- admission ----------------------------------------------------------
    def add(self, seq: Sequence) -> None:
        if self.config.debug_mode:
            self._check_new(seq)
        seq.block_size = self.block_size
        self.waiting.append(seq)

    def _check_new(self, seq: Sequence) -> None:
        queued = {s.seq_id for s in self.waiting} | {s.seq_id for s in self.running}
        if seq.status is not SequenceStatus.WAITING or seq.seq_id in queued:
            raise ValueError(f"request {seq.seq_id} is already admitted or finished")
        if seq.max_tokens <= 0 or len(seq) >= self.max_length:
            raise ValueError(f"request {seq.seq_id}: prompt/generation length exceeds "
                             f"engine capacity ({self.max_length} tokens)")
        if seq.block_table:
            raise ValueError(f"request {seq.seq_id} already owns cache blocks")

    # -- one step -----------------------------------------------------------
    def schedule(self) -> tuple[list[Sequence], bool]:
        """The requests of the next step and whether any of them prefills."""
        if self._inflight is not None:
            raise RuntimeError("the previous step has not been postprocessed")
        if self.is_finished():
            return [], True
        while True:
            step = _StepBuilder(self.max_num_batched_tokens, self.max_num_seqs)
            if self.config.mixed_batch:
                self._decode_pass(step)
                self._prompt_pass(step)
            else:
                self._prompt_pass(step)
                if not step.entries:
                    self._decode_pass(step)
            if step.entries:
                break
            # Decode pressure can have evicted requests into the waiting
            # queue; if its head fits now, build the step again.
            if not self.waiting or self.block_manager.can_allocate(self.waiting[0]) < 0:
                raise RuntimeError("KV cache cannot make progress")
        seqs = step.entries
        n_prefill = sum(1 for s in seqs if s.is_prefill)
        self._count_step(n_prefill, len(seqs))
        self._inflight = (seqs, n_prefill > 0)
        return seqs, n_prefill > 0

    def _count_step(self, n_prefill: int, n_total: int) -> None:
        self._counts["num_steps"] += 1
        if n_prefill == 0:
            kind = "num_decode_steps"
        elif n_prefill == n_total:
            kind = "num_prefill_steps"
        else:
            kind = "num_mixed_steps"
        self._counts[kind] += 1

    def _decode_pass(self, step: _StepBuilder) -> None:
        """One token for each running request, oldest first, while room lasts."""
        served: list[Sequence] = []
        pending = len(self.running)
        while pending and self.running and step.has_room():
            pending -= 1
            seq = self.running.popleft()
            if not self._secure_next_slot(seq):
                continue  # it evicted itself
            self.block_manager.may_append(seq)
            step.add(seq, 1, prefill=False)
            served.append(seq)
        self.running.extend(served)

    def _secure_next_slot(self, seq: Sequence) -> bool:
        """Evict the newest running requests until ``seq`` can append a token.

        Returns False when ``seq`` itself had to be evicted.
        """
        manager = self.block_manager
        while not manager.can_append(seq):
            victim = self.running.pop() if self.running else seq
            self.preempt(victim)
            if victim is seq:
                return False
        return True

    def _prompt_pass(self, step: _StepBuilder) -> None:
        """Prompt chunks in arrival order; a chunk short of its prompt ends the pass."""
        manager = self.block_manager
        while self.waiting and step.has_room():
            seq = self.waiting[0]
            if seq.block_table:
                start = seq.num_cached_tokens
                reuse = None
            else:
                reuse = manager.can_allocate(seq)
                if reuse < 0:
                    return  # the cache cannot hold it yet
                start = reuse * self.block_size
            left = seq.num_tokens - start
            if left <= 0:
                return
            chunk = min(left, step.tokens, self.config.max_num_prefill_tokens)
            if reuse is not None:
                manager.allocate(seq, reuse)
            step.add(seq, chunk, prefill=True)
            if seq.num_cached_tokens + chunk == seq.num_tokens:
                self.waiting.popleft()
                seq.start_running()
                self.running.append(seq)
            if chunk < left:
                return

    # -- eviction, completion, abort ------------------------------------------
    def preempt(self, seq: Sequence) -> None:
        """Free ``seq``'s blocks and put it at the front of the waiting queue."""
        self._counts["num_preemptions"] += 1
        seq.requeue()
        self.block_manager.deallocate(seq)
        self.waiting.appendleft(seq)

    def postprocess(self, seqs: list[Sequence], token_ids: list[int], is_prefill: bool) -> None:
        if self.config.debug_mode:
            if self._inflight != (seqs, is_prefill) or len(seqs) != len(token_ids):
                raise ValueError("postprocess call does not match the scheduled step")
            bad = [t for t in token_ids if type(t) is not int or t < 0]
            if bad:
                raise ValueError(f"invalid sampled token ids {bad}")
        for seq, token in zip(seqs, token_ids):
            self._commit(seq, token, is_prefill)
        self._inflight = None

    def _commit(self, seq: Sequence, token: int, is_prefill: bool) -> None:
        self.block_manager.hash_blocks(seq)
        seq.num_cached_tokens += seq.num_scheduled_tokens
        seq.num_scheduled_tokens = 0
        if is_prefill and seq.num_cached_tokens < seq.num_tokens:
            return  # a prompt chunk that stops short of the prompt's end samples nothing
        seq.append_token(token)
        reason = None
        if token == self.eos and not seq.ignore_eos:
            reason = "eos"
        elif seq.num_completion_tokens >= seq.max_tokens or len(seq) >= self.max_length:
            reason = "length"
        if reason is not None:
            seq.finish(reason)
            self.block_manager.deallocate(seq)
            self.running.remove(seq)

    def abort(self, seq_id: int) -> bool:
        """Finish request ``seq_id`` wherever it is queued; False if unknown."""
        for queue in (self.waiting, self.running):
            seq = next((s for s in queue if s.seq_id == seq_id), None)
            if seq is None:
                continue
            queue.remove(seq)
            self.block_manager.deallocate(seq)
            seq.finish("abort")
            if self._inflight is not None:
                kept = [s for s in self._inflight[0] if s.seq_id != seq_id]
                self._inflight = (kept, self._inflight[1]) if kept else None
            return True
        return False

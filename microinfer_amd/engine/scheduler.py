"""Step scheduling: decode first, then chunked prefill in the leftover budget.

Mirrors ``Scheduler`` (microinfer/engine/scheduler.py:8-260) without the
speculative-decoding hooks. The policy the reference's tests pin
(tests/components/test_scheduler.py) is kept exactly:

* with ``mixed_batch`` every running sequence gets one decode token first
  (round-robin when the token budget runs out), then waiting prompts fill the
  rest of ``max_num_batched_tokens`` in arrival order, each chunk capped by
  ``max_num_prefill_tokens``; a partly scheduled prompt ends the step's
  prefill. Without it, prefill runs first and decode only when nothing is
  waiting;
* a running sequence that cannot get a block preempts the newest running
  sequence (or itself): its blocks are freed and it returns to the front of
  the waiting queue with all its tokens, to be prefilled again;
* ``postprocess`` publishes completed blocks, advances the cached count,
  drops the sample of an unfinished prefill chunk and applies the EOS and
  length limits.
"""

from __future__ import annotations

from collections import deque

from microinfer_amd.engine.blockmanager import BlockManager
from microinfer_amd.engine.config import EngineConfig
from microinfer_amd.engine.sequence import Sequence, SequenceStatus


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
        self._inflight: tuple[list[Sequence], bool] | None = None
        self.num_preemptions = 0
        self.num_steps = 0
        self.num_prefill_steps = 0
        self.num_decode_steps = 0
        self.num_mixed_steps = 0

    @property
    def max_length(self) -> int:
        return min(self.config.max_model_len, len(self.block_manager.blocks) * self.block_size)

    def is_finished(self) -> bool:
        return not self.waiting and not self.running

    def stats(self) -> dict:
        return {
            "waiting": len(self.waiting),
            "running": len(self.running),
            "num_preemptions": self.num_preemptions,
            "num_steps": self.num_steps,
            "num_prefill_steps": self.num_prefill_steps,
            "num_decode_steps": self.num_decode_steps,
            "num_mixed_steps": self.num_mixed_steps,
        }

    def add(self, seq: Sequence) -> None:
        if self.config.debug_mode:
            known = any(s.seq_id == seq.seq_id for s in (*self.waiting, *self.running))
            if seq.status != SequenceStatus.WAITING or known:
                raise ValueError("request already admitted or finished")
            if seq.max_tokens <= 0 or len(seq) >= self.max_length:
                raise ValueError("prompt/generation length exceeds engine capacity")
            if seq.block_table:
                raise ValueError("new request already owns cache blocks")
        seq.block_size = self.block_size
        self.waiting.append(seq)

    def schedule(self) -> tuple[list[Sequence], bool]:
        """The sequences of the next step and whether any of them prefills."""
        if self._inflight is not None:
            raise RuntimeError("previous schedule has not been postprocessed")
        if self.is_finished():
            return [], True
        budget = self.max_num_batched_tokens
        if self.config.mixed_batch:
            seqs, budget = self._schedule_decode(budget)
            seqs += self._schedule_prefill(budget, len(seqs))
        else:
            seqs = self._schedule_prefill(budget, 0)
            if not seqs:
                seqs, _ = self._schedule_decode(budget)
        if not seqs:
            # Decode pressure may have preempted into the waiting queue; retry
            # if its head now fits, otherwise nothing can ever run.
            if self.waiting and self.block_manager.can_allocate(self.waiting[0]) >= 0:
                return self.schedule()
            raise RuntimeError("KV cache cannot make progress")
        prefills = sum(seq.is_prefill for seq in seqs)
        self.num_steps += 1
        if prefills and prefills < len(seqs):
            self.num_mixed_steps += 1
        elif prefills:
            self.num_prefill_steps += 1
        else:
            self.num_decode_steps += 1
        self._inflight = (seqs, prefills > 0)
        return seqs, prefills > 0

    def _schedule_decode(self, budget: int) -> tuple[list[Sequence], int]:
        chosen: list[Sequence] = []
        for _ in range(len(self.running)):
            if not self.running or len(chosen) >= self.max_num_seqs or budget <= 0:
                break
            seq = self.running.popleft()
            while not self.block_manager.can_append(seq):
                if self.running:
                    self.preempt(self.running.pop())
                else:
                    self.preempt(seq)
                    seq = None
                    break
            if seq is None:
                continue
            seq.num_scheduled_tokens = 1
            seq.is_prefill = False
            self.block_manager.may_append(seq)
            chosen.append(seq)
            budget -= 1
        # Served sequences go to the back, so a short budget rotates through all.
        self.running.extend(chosen)
        return chosen, budget

    def _schedule_prefill(self, budget: int, already: int) -> list[Sequence]:
        chosen: list[Sequence] = []
        while self.waiting and already + len(chosen) < self.max_num_seqs and budget > 0:
            seq = self.waiting[0]
            fresh = not seq.block_table
            if fresh:
                cached_blocks = self.block_manager.can_allocate(seq)
                if cached_blocks < 0:
                    break
                remaining = seq.num_tokens - cached_blocks * self.block_size
            else:
                remaining = seq.num_tokens - seq.num_cached_tokens
            if remaining <= 0:
                break
            take = min(remaining, budget, self.config.max_num_prefill_tokens)
            if fresh:
                self.block_manager.allocate(seq, cached_blocks)
            seq.num_scheduled_tokens = take
            seq.is_prefill = True
            budget -= take
            if seq.num_cached_tokens + take == seq.num_tokens:
                seq.status = SequenceStatus.RUNNING
                self.waiting.popleft()
                self.running.append(seq)
            chosen.append(seq)
            if take < remaining:
                break  # one partial chunk per step
        return chosen

    def preempt(self, seq: Sequence) -> None:
        self.num_preemptions += 1
        seq.status = SequenceStatus.WAITING
        seq.is_prefill = True
        seq.num_scheduled_tokens = 0
        self.block_manager.deallocate(seq)
        self.waiting.appendleft(seq)

    def postprocess(self, seqs: list[Sequence], token_ids: list[int], is_prefill: bool) -> None:
        if self.config.debug_mode:
            if self._inflight != (seqs, is_prefill) or len(seqs) != len(token_ids):
                raise ValueError("postprocess does not match scheduled work")
            if any(type(t) is not int or t < 0 for t in token_ids):
                raise ValueError("invalid sampled token")
        for seq, token in zip(seqs, token_ids):
            self.block_manager.hash_blocks(seq)
            seq.num_cached_tokens += seq.num_scheduled_tokens
            seq.num_scheduled_tokens = 0
            if is_prefill and seq.num_cached_tokens < seq.num_tokens:
                continue  # a prompt chunk short of the end samples nothing
            seq.append_token(token)
            if not seq.ignore_eos and token == self.eos:
                seq.finish_reason = "eos"
            elif seq.num_completion_tokens >= seq.max_tokens or len(seq) >= self.max_length:
                seq.finish_reason = "length"
            if seq.finish_reason is not None:
                seq.status = SequenceStatus.FINISHED
                self.block_manager.deallocate(seq)
                self.running.remove(seq)
        self._inflight = None

    def abort(self, seq_id: int) -> bool:
        for queue in (self.waiting, self.running):
            for seq in queue:
                if seq.seq_id != seq_id:
                    continue
                queue.remove(seq)
                self.block_manager.deallocate(seq)
                seq.num_scheduled_tokens = 0
                seq.status = SequenceStatus.FINISHED
                seq.finish_reason = "abort"
                if self._inflight is not None:
                    rest = [s for s in self._inflight[0] if s.seq_id != seq_id]
                    self._inflight = (rest, self._inflight[1]) if rest else None
                return True
        return False

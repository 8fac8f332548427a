"""The step loop: schedule, run, postprocess.

Mirrors ``LLMEngine`` (microinfer/engine/llm_engine.py:5-94, :226-238)
without speculative decoding: a mixed step runs its decode rows (graph path)
and its prefill rows as two model calls and merges the tokens in schedule
order; a failing model call aborts every scheduled request before any block
hash is published, then re-raises.
"""

from __future__ import annotations

from microinfer_amd.engine.sequence import Sequence, SequenceStatus


class LLMEngine:
    def __init__(self, scheduler, runner):
        self.scheduler, self.model_runner = scheduler, runner

    def add_request(self, seq: Sequence) -> None:
        self.scheduler.add(seq)

    def is_finished(self) -> bool:
        return self.scheduler.is_finished()

    def step(self):
        """``(finished, num_tokens)``: finished ``(seq_id, completion)`` pairs
        and the step's token count (negative for a decode-only step)."""
        finished, num_tokens, _ = self.step_events()
        return finished, num_tokens

    def step_events(self):
        seqs, prefill = self.scheduler.schedule()
        if not seqs:
            return [], 0, []
        num_tokens = sum(s.num_scheduled_tokens for s in seqs) if prefill else -len(seqs)
        try:
            decode = [s for s in seqs if not s.is_prefill]
            if prefill and decode:
                chunks = [s for s in seqs if s.is_prefill]
                by_id = dict(zip((s.seq_id for s in decode),
                                 self.model_runner.run(decode, False)))
                by_id.update(zip((s.seq_id for s in chunks), self.model_runner.run(chunks, True)))
                tokens = [by_id[s.seq_id] for s in seqs]
            else:
                tokens = self.model_runner.run(seqs, prefill)
        except Exception:
            for seq in seqs:  # KV may be partly written: publish nothing
                self.scheduler.abort(seq.seq_id)
            raise
        self.scheduler.postprocess(seqs, tokens, prefill)
        done = [s.status == SequenceStatus.FINISHED for s in seqs]
        finished = [(s.seq_id, s.completion_token_ids) for s, d in zip(seqs, done) if d]
        updates = [(s.seq_id, tuple(s.completion_token_ids), d, s.finish_reason)
                   for s, d in zip(seqs, done)]
        return finished, num_tokens, updates

    def stats(self) -> dict:
        stats = self.scheduler.stats()
        stats.update(self.scheduler.block_manager.stats())
        return stats

    def abort(self, seq_id: int) -> bool:
        return self.scheduler.abort(seq_id)

    def generate(self, prompts, sampling_params) -> list[list[int]]:
        """Run requests to completion; completions in prompt order."""
        params = (sampling_params if isinstance(sampling_params, list)
                  else [sampling_params] * len(prompts))
        seqs = [Sequence(list(p), sp) for p, sp in zip(prompts, params)]
        for seq in seqs:
            self.add_request(seq)
        while not self.is_finished():
            self.step()
        return [seq.completion_token_ids for seq in seqs]

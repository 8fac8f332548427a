"""The engine's step loop with a stand-in runner (CPU, no kernels).

``LLMEngine`` (mirroring microinfer/engine/llm_engine.py:25-94): a mixed
step calls the runner for its decode rows and its prefill rows separately
and merges the tokens in schedule order; a failing runner call aborts every
scheduled request, frees their blocks and re-raises; ``generate`` runs
requests to completion.
"""

import pytest

from microinfer_amd.engine.config import SampleParameter
from microinfer_amd.engine.llm_engine import LLMEngine
from microinfer_amd.engine.sequence import SequenceStatus


class CountingRunner:
    """Returns 100 + (sequence length) for every row and records calls."""

    def __init__(self):
        self.calls = []
        self.fail = False

    def run(self, seqs, is_prefill):
        if self.fail:
            raise RuntimeError("device error")
        self.calls.append(([s.seq_id for s in seqs], is_prefill))
        return [100 + len(s) for s in seqs]


def test_mixed_step_runs_decode_and_prefill_separately(scheduler_factory, sequence_cls):
    scheduler, _ = scheduler_factory(max_num_batched_tokens=4)
    runner = CountingRunner()
    engine = LLMEngine(scheduler, runner)
    a = sequence_cls([1], SampleParameter(max_tokens=3))
    engine.add_request(a)
    engine.step()
    b = sequence_cls([5, 6], SampleParameter(max_tokens=1))
    engine.add_request(b)
    finished, num_tokens, updates = engine.step_events()
    assert runner.calls[-2:] == [([a.seq_id], False), ([b.seq_id], True)]
    assert num_tokens == 3
    assert a.completion_token_ids == [101, 102] and b.completion_token_ids == [102]
    assert finished == [(b.seq_id, [102])]
    assert [u[0] for u in updates] == [a.seq_id, b.seq_id] and updates[1][2]
    finished, num_tokens = engine.step()
    assert num_tokens == -1 and finished == [(a.seq_id, [101, 102, 103])]
    assert engine.is_finished()
    assert engine.stats()["num_mixed_steps"] == 1


def test_runner_failure_aborts_the_step(scheduler_factory, sequence_cls):
    scheduler, manager = scheduler_factory()
    runner = CountingRunner()
    engine = LLMEngine(scheduler, runner)
    seqs = [sequence_cls([1, 2, 3]), sequence_cls([4, 5])]
    for s in seqs:
        engine.add_request(s)
    runner.fail = True
    with pytest.raises(RuntimeError, match="device error"):
        engine.step()
    assert all(s.status == SequenceStatus.FINISHED and s.finish_reason == "abort" for s in seqs)
    assert not manager.used_block_ids and not manager.hash_to_block_id
    assert engine.is_finished()
    assert not engine.abort(seqs[0].seq_id)


def test_generate_returns_completions_in_prompt_order(scheduler_factory):
    scheduler, manager = scheduler_factory(max_num_batched_tokens=5)
    engine = LLMEngine(scheduler, CountingRunner())
    out = engine.generate([[1, 2, 3], [4], [5, 6, 7, 8, 9, 10]], SampleParameter(max_tokens=2))
    assert out == [[103, 104], [101, 102], [106, 107]]
    assert not manager.used_block_ids

"""Step scheduling (microinfer_amd.engine.scheduler).

The cases and expected values are the reference's own
(tests/components/test_scheduler.py), run against this engine with 4-token
blocks: lazy admission, chunked prefill that discards the intermediate
sample, mixed decode + prefill steps, the prefill chunk cap, the prefill-first
policy, arrival order, sequence and token limits, prefix reuse, EOS, and
preemption under decode pressure.
"""

import pytest

from microinfer_amd.engine.config import EngineConfig, SampleParameter
from microinfer_amd.engine.sequence import SequenceStatus


def step(scheduler, tokens):
    seqs, prefill = scheduler.schedule()
    scheduler.postprocess(seqs, tokens, prefill)
    return seqs, prefill


def test_config_validation():
    for bad in (dict(max_num_seqs=0), dict(max_model_len=1.5), dict(eos_token_id=-1),
                dict(mixed_batch=1)):
        with pytest.raises(ValueError):
            EngineConfig(**bad)


def test_empty_and_lazy_admission(scheduler_factory, sequence_cls):
    scheduler, manager = scheduler_factory()
    assert scheduler.is_finished()
    seq = sequence_cls([1, 2])
    scheduler.add(seq)
    assert not scheduler.is_finished()
    assert not seq.block_table and not manager.used_block_ids


def test_chunked_prefill_drops_the_intermediate_sample(scheduler_factory, sequence_cls):
    scheduler, manager = scheduler_factory(max_num_batched_tokens=3)
    seq = sequence_cls([1, 2, 3, 4, 5], SampleParameter(max_tokens=2))
    scheduler.add(seq)
    seqs, prefill = scheduler.schedule()
    assert prefill is True and seqs == [seq]
    assert (seq.num_scheduled_tokens, seq.num_cached_tokens) == (3, 0)
    assert seq.status == SequenceStatus.WAITING and not manager.hash_to_block_id
    scheduler.postprocess(seqs, [99], prefill)
    assert seq.token_ids == [1, 2, 3, 4, 5]
    assert (seq.num_cached_tokens, seq.num_scheduled_tokens) == (3, 0)
    seqs, prefill = scheduler.schedule()
    assert prefill and seq.num_scheduled_tokens == 2 and seq.status == SequenceStatus.RUNNING
    scheduler.postprocess(seqs, [6], prefill)
    assert seq.completion_token_ids == [6] and seq.num_cached_tokens == 5
    assert manager.compute_hash([1, 2, 3, 4]) in manager.hash_to_block_id
    seqs, prefill = scheduler.schedule()
    assert prefill is False and seq.num_scheduled_tokens == 1
    scheduler.postprocess(seqs, [7], prefill)
    assert seq.is_finished and seq.completion_token_ids == [6, 7]
    assert not manager.used_block_ids and scheduler.is_finished()


def test_running_decode_mixes_with_waiting_prefill(scheduler_factory, sequence_cls):
    scheduler, _ = scheduler_factory(max_num_batched_tokens=4)
    a = sequence_cls([1])
    scheduler.add(a)
    step(scheduler, [2])
    b = sequence_cls([5, 6])
    scheduler.add(b)
    seqs, prefill = scheduler.schedule()
    assert prefill is True and seqs == [a, b]
    assert a.num_scheduled_tokens == 1 and not a.is_prefill
    assert b.num_scheduled_tokens == 2 and b.is_prefill
    assert scheduler.num_mixed_steps == 1


def test_prefill_chunk_cap(scheduler_factory, sequence_cls):
    scheduler, _ = scheduler_factory(max_num_batched_tokens=16, max_num_prefill_tokens=3)
    seq = sequence_cls(list(range(8)))
    scheduler.add(seq)
    seqs, prefill = scheduler.schedule()
    assert prefill and seqs == [seq] and seq.num_scheduled_tokens == 3
    assert seq.status == SequenceStatus.WAITING


def test_prefill_first_policy(scheduler_factory, sequence_cls):
    scheduler, _ = scheduler_factory(max_num_batched_tokens=4, mixed_batch=False)
    a = sequence_cls([1])
    scheduler.add(a)
    step(scheduler, [2])
    b = sequence_cls([5, 6])
    scheduler.add(b)
    seqs, prefill = scheduler.schedule()
    assert prefill is True and seqs == [b]
    assert a.num_scheduled_tokens == 0 and a.completion_token_ids == [2]


def test_prefill_fills_the_budget_in_arrival_order(scheduler_factory, sequence_cls):
    scheduler, _ = scheduler_factory(max_num_batched_tokens=4)
    a, b = sequence_cls([1, 2]), sequence_cls([3, 4, 5])
    scheduler.add(a)
    scheduler.add(b)
    seqs, prefill = scheduler.schedule()
    assert prefill and seqs == [a, b]
    assert a.num_scheduled_tokens == 2 and a.status == SequenceStatus.RUNNING
    assert b.num_scheduled_tokens == 2 and b.status == SequenceStatus.WAITING
    assert b.num_cached_tokens == 0
    scheduler.postprocess(seqs, [10, 11], prefill)
    assert b.num_cached_tokens == 2 and b.completion_token_ids == []
    seqs, prefill = scheduler.schedule()
    assert prefill and seqs == [a, b]
    assert a.num_scheduled_tokens == 1 and b.num_scheduled_tokens == 1


def test_sequence_limit_and_fcfs(scheduler_factory, sequence_cls):
    scheduler, _ = scheduler_factory(max_num_seqs=1)
    a, b = [sequence_cls([i], SampleParameter(max_tokens=1)) for i in (1, 2)]
    scheduler.add(a)
    scheduler.add(b)
    seqs, prefill = scheduler.schedule()
    assert seqs == [a] and prefill
    scheduler.postprocess(seqs, [3], prefill)
    assert scheduler.schedule()[0] == [b]


def test_decode_token_budget_rotates(scheduler_factory, sequence_cls):
    scheduler, _ = scheduler_factory(max_num_batched_tokens=2, max_num_seqs=2)
    a, b = sequence_cls([1]), sequence_cls([3])
    scheduler.add(a)
    scheduler.add(b)
    step(scheduler, [2, 4])
    scheduler.max_num_batched_tokens = 1
    seqs, prefill = scheduler.schedule()
    assert not prefill and seqs == [a] and a.num_scheduled_tokens == 1
    scheduler.postprocess(seqs, [5], prefill)
    assert scheduler.schedule()[0] == [b]


def test_completed_prefix_is_reused(scheduler_factory, sequence_cls):
    scheduler, manager = scheduler_factory()
    a = sequence_cls([1, 2, 3, 4, 5], SampleParameter(max_tokens=1))
    scheduler.add(a)
    seqs, prefill = scheduler.schedule()
    old = a.block_table[0]
    scheduler.postprocess(seqs, [9], prefill)
    b = sequence_cls([1, 2, 3, 4, 6])
    scheduler.add(b)
    seqs, prefill = scheduler.schedule()
    assert prefill and seqs == [b]
    assert (b.num_cached_tokens, b.num_scheduled_tokens) == (4, 1)
    assert b.block_table[0] == old and manager.blocks[old].ref_count == 1


@pytest.mark.parametrize("ignore_eos,finished", [(False, True), (True, False)])
def test_eos(scheduler_factory, sequence_cls, ignore_eos, finished):
    scheduler, _ = scheduler_factory()
    seq = sequence_cls([1], SampleParameter(ignore_eos=ignore_eos))
    scheduler.add(seq)
    step(scheduler, [0])
    assert seq.is_finished == finished and seq.completion_token_ids == [0]
    assert seq.finish_reason == ("eos" if finished else None)


def test_preempted_sequence_keeps_tokens_and_goes_first(scheduler_factory, sequence_cls):
    scheduler, _ = scheduler_factory()
    seq = sequence_cls([1, 2, 3, 4, 5])
    scheduler.add(seq)
    step(scheduler, [6])
    scheduler.running.remove(seq)
    scheduler.preempt(seq)
    assert seq.token_ids == [1, 2, 3, 4, 5, 6]
    assert seq.num_cached_tokens == 0 and not seq.block_table
    assert seq.status == SequenceStatus.WAITING and seq.is_prefill
    assert scheduler.waiting[0] is seq
    step(scheduler, [7])
    assert seq.completion_token_ids == [6, 7]


def test_decode_pressure_preempts_the_newest(scheduler_factory, sequence_cls):
    scheduler, manager = scheduler_factory(num_blocks=2)
    a = sequence_cls([1, 2, 3, 4], SampleParameter(max_tokens=2))
    b = sequence_cls([7, 8, 9, 10], SampleParameter(max_tokens=2))
    scheduler.add(a)
    scheduler.add(b)
    step(scheduler, [5, 11])
    seqs, prefill = scheduler.schedule()
    assert not prefill and seqs == [a]
    assert b.status == SequenceStatus.WAITING and not b.block_table
    assert scheduler.num_preemptions == 1
    scheduler.postprocess(seqs, [6], prefill)
    step(scheduler, [12])
    assert b.completion_token_ids == [11, 12]
    assert scheduler.is_finished() and not manager.used_block_ids


def test_length_limit_and_abort(scheduler_factory, sequence_cls):
    scheduler, manager = scheduler_factory(max_model_len=6)
    a = sequence_cls([1, 2, 3, 4, 5])
    b = sequence_cls([8, 9])
    scheduler.add(a)
    scheduler.add(b)
    seqs, prefill = scheduler.schedule()
    assert scheduler.abort(b.seq_id) and b.finish_reason == "abort"
    scheduler.postprocess([a], [6], prefill)
    assert a.is_finished and a.finish_reason == "length" and len(a) == 6
    assert not scheduler.abort(12345)
    assert scheduler.is_finished() and not manager.used_block_ids


def test_schedule_twice_without_postprocess_fails(scheduler_factory, sequence_cls):
    scheduler, _ = scheduler_factory()
    scheduler.add(sequence_cls([1, 2]))
    scheduler.schedule()
    with pytest.raises(RuntimeError, match="postprocessed"):
        scheduler.schedule()


def test_debug_mode_checks(scheduler_factory, sequence_cls):
    scheduler, _ = scheduler_factory(debug_mode=True, max_model_len=8)
    seq = sequence_cls([1, 2])
    scheduler.add(seq)
    with pytest.raises(ValueError, match="already"):
        scheduler.add(seq)
    with pytest.raises(ValueError, match="exceeds"):
        scheduler.add(sequence_cls(list(range(8))))
    seqs, prefill = scheduler.schedule()
    with pytest.raises(ValueError, match="does not match"):
        scheduler.postprocess(seqs, [1, 2], prefill)
    with pytest.raises(ValueError, match="invalid"):
        scheduler.postprocess(seqs, [-1], prefill)

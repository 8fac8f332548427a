"""Block ownership and prefix caching (microinfer_amd.engine.blockmanager).

The cases and expected values are the reference's own
(tests/engine/test_blockmanager.py and tests/engine/test_sequence.py), run
against this engine's Sequence and BlockManager with 4-token blocks.
"""

from collections import Counter

import pytest

from microinfer_amd.engine.blockmanager import Block, BlockManager
from microinfer_amd.engine.config import SampleParameter
from microinfer_amd.engine.sequence import SequenceStatus


def owners_agree(manager, *seqs):
    refs = Counter(b for s in seqs for b in s.block_table)
    free = list(manager.free_block_ids)
    used = manager.used_block_ids
    assert len(free) == len(set(free)) and set(free).isdisjoint(used)
    assert set(free) | used == set(range(len(manager.blocks)))
    assert used == set(refs)
    assert all(b.ref_count == refs[b.block_id] for b in manager.blocks)


def mark_cached(manager, seq, count):
    """Publish the first ``count`` full blocks as hash_blocks would."""
    prefix = -1
    for i in range(count):
        tokens = seq.block(i)
        prefix = manager.compute_hash(tokens, prefix)
        manager.blocks[seq.block_table[i]].update(prefix, tokens)
        manager.hash_to_block_id[prefix] = seq.block_table[i]


# -- Sequence (test_sequence.py) ---------------------------------------------

def test_sequence_copies_tokens_and_sampling_values(sequence_cls):
    tokens = [1, 2, 3]
    seq = sequence_cls(tokens, SampleParameter(0.5, 7, True))
    tokens.append(99)
    assert seq.token_ids == [1, 2, 3] and seq.status == SequenceStatus.WAITING
    assert not seq.is_finished
    assert (seq.temperature, seq.max_tokens, seq.ignore_eos) == (0.5, 7, True)
    assert seq.seq_id != sequence_cls([1]).seq_id
    with pytest.raises(ValueError):
        sequence_cls([])
    with pytest.raises(ValueError):
        sequence_cls([1, -2])


@pytest.mark.parametrize("length", [1, 3, 4, 5, 8, 9])
def test_sequence_blocks_partition_the_tokens(sequence_cls, length):
    seq = sequence_cls(list(range(length)))
    chunks = [seq.block(i) for i in range(seq.num_blocks)]
    assert sum(chunks, []) == seq.token_ids
    assert all(len(c) == 4 for c in chunks[:-1]) and len(chunks[-1]) == seq.last_block_num_tokens
    assert seq.num_blocks == (length + 3) // 4
    for bad in (-1, seq.num_blocks):
        with pytest.raises(AssertionError):
            seq.block(bad)


def test_sequence_append_tracks_completion(sequence_cls):
    seq = sequence_cls([1, 2, 3, 4])
    seq.append_token(5)
    seq.append_token(6)
    assert len(seq) == 6 and seq.last_token == seq[-1] == 6
    assert seq.prompt_token_ids == [1, 2, 3, 4] and seq.completion_token_ids == [5, 6]
    assert seq.num_completion_tokens == 2


def test_sample_parameter_validation():
    with pytest.raises(AssertionError):
        SampleParameter(temperature=0.0)
    with pytest.raises(ValueError):
        SampleParameter(max_tokens=0)


# -- BlockManager (test_blockmanager.py) ---------------------------------------

def test_block_reset():
    block = Block(3)
    assert block.ref_count == 0
    block.update(123, [1, 2])
    block.reset()
    assert (block.block_id, block.ref_count, block.hash, block.token_ids) == (3, 1, -1, [])


def test_hash_chains_prefix_and_order():
    h = BlockManager.compute_hash
    assert h([1, 2]) == h([1, 2]) and h([1, 2]) != h([2, 1])
    assert h([1, 2], h([3, 4])) != h([1, 2], h([4, 3]))


def test_constructor_rejects_bad_sizes():
    for args in ((0, 4), (4, 0), (2.0, 4)):
        with pytest.raises(ValueError):
            BlockManager(*args)


@pytest.mark.parametrize("length", [1, 4, 5, 8, 9])
def test_allocate_then_release(sequence_cls, length):
    manager = BlockManager(3, 4)
    seq = sequence_cls(list(range(length)))
    assert manager.can_allocate(seq) == 0
    manager.allocate(seq, 0)
    assert len(seq.block_table) == seq.num_blocks
    assert not manager.hash_to_block_id
    owners_agree(manager, seq)
    manager.deallocate(seq)
    assert seq.block_table == [] and seq.num_cached_tokens == 0
    owners_agree(manager)


def test_capacity_check_changes_nothing(sequence_cls):
    manager = BlockManager(1, 4)
    assert manager.can_allocate(sequence_cls([1, 2, 3, 4, 5])) == -1
    owners_agree(manager)


def test_shared_prefix_outlives_first_owner(sequence_cls):
    manager = BlockManager(3, 4)
    a, b = sequence_cls([1, 2, 3, 4, 5]), sequence_cls([1, 2, 3, 4, 6])
    manager.allocate(a, 0)
    mark_cached(manager, a, 1)
    assert manager.can_allocate(b) == 1
    manager.allocate(b, 1)
    shared = a.block_table[0]
    assert b.block_table[0] == shared and b.num_cached_tokens == 4
    owners_agree(manager, a, b)
    manager.deallocate(a)
    assert shared not in manager.free_block_ids
    owners_agree(manager, b)
    manager.deallocate(b)
    owners_agree(manager)


def test_free_cached_prefix_is_taken_back(sequence_cls):
    manager = BlockManager(2, 4)
    a = sequence_cls([1, 2, 3, 4, 5])
    manager.allocate(a, 0)
    mark_cached(manager, a, 1)
    cached = a.block_table[0]
    manager.deallocate(a)
    b = sequence_cls([1, 2, 3, 4, 6])
    assert manager.can_allocate(b) == 1
    manager.allocate(b, 1)
    assert b.block_table[0] == cached
    owners_agree(manager, b)


@pytest.mark.parametrize("length", [3, 4, 8])
def test_last_block_never_comes_from_the_cache(sequence_cls, length):
    manager = BlockManager(4, 4)
    a = sequence_cls(list(range(length)))
    manager.allocate(a, 0)
    mark_cached(manager, a, length // 4)
    assert manager.can_allocate(sequence_cls(list(range(length)))) == a.num_blocks - 1


@pytest.mark.parametrize("length,grows", [(3, False), (4, True), (7, False), (8, True)])
def test_decode_append_at_block_boundary(sequence_cls, length, grows):
    manager = BlockManager(4, 4)
    seq = sequence_cls(list(range(length)))
    manager.allocate(seq, 0)
    before = list(seq.block_table)
    seq.append_token(99)
    assert manager.can_append(seq)
    manager.may_append(seq)
    assert len(seq.block_table) == len(before) + grows and seq.block_table[:len(before)] == before
    owners_agree(manager, seq)
    manager.deallocate(seq)
    owners_agree(manager)


def test_full_pool_refuses_append(sequence_cls):
    manager = BlockManager(1, 4)
    seq = sequence_cls([1, 2, 3, 4])
    manager.allocate(seq, 0)
    seq.append_token(5)
    assert not manager.can_append(seq)
    with pytest.raises(ValueError):
        manager.may_append(seq)
    manager.deallocate(seq)
    owners_agree(manager)


def test_free_cache_hit_is_not_extra_capacity(sequence_cls):
    manager = BlockManager(2, 4)
    cached = sequence_cls([1, 2, 3, 4])
    manager.allocate(cached, 0)
    mark_cached(manager, cached, 1)
    manager.deallocate(cached)
    busy = sequence_cls([9])
    manager.allocate(busy, 0)
    assert manager.can_allocate(sequence_cls([1, 2, 3, 4, 5])) == -1
    owners_agree(manager, busy)


def test_reuse_evicts_the_old_hash(sequence_cls):
    manager = BlockManager(1, 4)
    a = sequence_cls([1, 2, 3, 4])
    manager.allocate(a, 0)
    mark_cached(manager, a, 1)
    old = manager.compute_hash(a.token_ids)
    manager.deallocate(a)
    b = sequence_cls([8, 9, 10, 11])
    manager.allocate(b, 0)
    assert old not in manager.hash_to_block_id
    owners_agree(manager, b)


def test_reuse_keeps_a_hash_now_owned_by_another_block(sequence_cls):
    manager = BlockManager(2, 4)
    a, b = sequence_cls([1, 2, 3, 4]), sequence_cls([1, 2, 3, 4])
    for seq in (a, b):
        manager.allocate(seq, 0)
        mark_cached(manager, seq, 1)
    manager.deallocate(a)
    manager.allocate(sequence_cls([8]), 0)
    assert manager.hash_to_block_id[manager.compute_hash(b.token_ids)] == b.block_table[0]


def test_hash_hit_requires_equal_tokens(sequence_cls):
    manager = BlockManager(3, 4)
    a = sequence_cls([9, 9, 9, 9])
    manager.allocate(a, 0)
    manager.hash_to_block_id[manager.compute_hash([1, 2, 3, 4])] = a.block_table[0]
    assert manager.can_allocate(sequence_cls([1, 2, 3, 4, 5])) == 0


@pytest.mark.parametrize("scheduled", [0, 3, 4, 5, 8, 9])
def test_only_completed_blocks_are_published(sequence_cls, scheduled):
    manager = BlockManager(3, 4)
    seq = sequence_cls(list(range(9)))
    manager.allocate(seq, 0)
    seq.num_scheduled_tokens = scheduled
    manager.hash_blocks(seq)
    expected, prefix = {}, -1
    for i in range(scheduled // 4):
        prefix = manager.compute_hash(seq.block(i), prefix)
        expected[prefix] = seq.block_table[i]
    assert manager.hash_to_block_id == expected
    assert all(manager.blocks[b].hash == h for h, b in expected.items())


def test_chunked_prefill_publishes_for_reuse(sequence_cls):
    manager = BlockManager(5, 4)
    seq = sequence_cls(list(range(9)))
    manager.allocate(seq, 0)
    for chunk in (3, 2, 4):
        seq.num_scheduled_tokens = chunk
        manager.hash_blocks(seq)
        seq.num_cached_tokens += chunk
        seq.num_scheduled_tokens = 0
    second = sequence_cls(list(range(8)) + [99])
    assert manager.can_allocate(second) == 2
    manager.allocate(second, 2)
    assert second.block_table[:2] == seq.block_table[:2]
    owners_agree(manager, seq, second)


def test_decode_token_completes_and_publishes_a_block(sequence_cls):
    manager = BlockManager(2, 4)
    seq = sequence_cls([1, 2, 3])
    manager.allocate(seq, 0)
    seq.num_cached_tokens = 3
    seq.append_token(4)
    manager.may_append(seq)
    seq.num_scheduled_tokens = 1
    manager.hash_blocks(seq)
    bid, key = seq.block_table[0], manager.compute_hash([1, 2, 3, 4])
    assert manager.hash_to_block_id == {key: bid}
    assert manager.blocks[bid].token_ids == [1, 2, 3, 4] and manager.blocks[bid].hash == key


def test_free_blocks_are_reused_least_recent_first(sequence_cls):
    manager = BlockManager(3, 4)
    seqs = [sequence_cls(t) for t in ([1, 2, 3, 4], [11, 12, 13, 14], [21, 22, 23, 24])]
    for seq in seqs:
        manager.allocate(seq, 0)
        mark_cached(manager, seq, 1)
    ids = [seq.block_table[0] for seq in seqs]
    for seq in seqs:
        manager.deallocate(seq)
    assert manager.can_allocate(sequence_cls([1, 2, 3, 4, 99])) == 1  # refreshes ids[0]
    fresh = sequence_cls(list(range(31, 39)))
    manager.allocate(fresh, 0)
    assert fresh.block_table == ids[1:] and ids[0] not in fresh.block_table
    assert manager.stats()["prefix_cache_evictions"] == 2


def test_prefix_cache_statistics(sequence_cls):
    manager = BlockManager(3, 4)
    a = sequence_cls([1, 2, 3, 4, 5])
    manager.allocate(a, 0)
    mark_cached(manager, a, 1)
    manager.deallocate(a)
    b = sequence_cls([1, 2, 3, 4, 6])
    assert manager.can_allocate(b) == 1
    manager.allocate(b, 1)
    stats = manager.stats()
    assert (stats["prefix_cache_hit_tokens"], stats["prefix_cache_hit_blocks"],
            stats["prefix_cache_entries"]) == (4, 1, 1)


def test_prefix_cache_reset_needs_an_idle_pool(sequence_cls):
    manager = BlockManager(2, 4)
    seq = sequence_cls([1, 2, 3, 4])
    manager.allocate(seq, 0)
    with pytest.raises(RuntimeError, match="in use"):
        manager.reset_prefix_cache()
    manager.deallocate(seq)
    manager.blocks[0].update(123, [1, 2, 3, 4])
    manager.hash_to_block_id[123] = 0
    manager.prefix_cache_hit_tokens = 4
    manager.reset_prefix_cache()
    assert manager.hash_to_block_id == {} and manager.prefix_cache_hit_tokens == 0
    assert all(b.hash == -1 and b.token_ids == [] for b in manager.blocks)


def test_trim_releases_blocks_past_the_length(sequence_cls):
    manager = BlockManager(4, 4)
    seq = sequence_cls(list(range(9)))
    manager.allocate(seq, 0)
    seq.token_ids = seq.token_ids[:4]
    seq.num_tokens = 4
    manager.trim(seq)
    assert len(seq.block_table) == 1
    owners_agree(manager, seq)

"""Pin the append, slot and gather restatements against the reference's known answers."""

import numpy as np
import pytest

from microinfer_amd.workloads import decode_slots, draw_tables, make_decode_batch
from oracle import gather_paged_kv, kv_append, slot_indices


def test_append_then_gather_known_answer():
    # test_kv_cache.py:10-23: arange(30) into slots [8, 9, 10, 11, 0] (B = 4),
    # read back through table [2, 0]; other blocks keep their fill.
    keys_cache = np.full((3, 4, 2, 3), -5.0, np.float32)
    values_cache = np.full_like(keys_cache, -6.0)
    keys = np.arange(30, dtype=np.float32).reshape(5, 2, 3)
    values = keys + 100
    kv_append(keys_cache, values_cache, [8, 9, 10, 11, 0], keys, values)
    k, v = gather_paged_kv(keys_cache, values_cache, [[2, 0]], [5], 4)
    np.testing.assert_array_equal(k, keys)
    np.testing.assert_array_equal(v, values)
    assert (keys_cache[1] == -5).all()


def test_padding_slot_is_skipped():
    # test_kv_cache.py:26-32.
    cache_k = np.full((2, 4, 1, 2), 9.0, np.float32)
    cache_v = np.full_like(cache_k, 9.0)
    kv_append(cache_k, cache_v, [-1, 0], np.zeros((2, 1, 2)), np.ones((2, 1, 2)))
    assert (cache_k[0, -1, -1] == 9).all() and (cache_k[-1, -1, -1] == 9).all()
    assert (cache_k[0, 0, 0] == 0).all() and (cache_v[0, 0, 0] == 1).all()


def test_append_is_bit_exact_on_raw_bf16_patterns():
    rng = np.random.default_rng(0)
    cache_k = rng.integers(0, 1 << 16, (4, 4, 2, 8), dtype=np.uint16)
    cache_v = cache_k.copy()
    rows = rng.integers(0, 1 << 16, (3, 2, 8), dtype=np.uint16)
    before = cache_k.copy()
    kv_append(cache_k, cache_v, [13, 2, 7], rows, rows)
    for slot, row in zip([13, 2, 7], rows):
        assert np.array_equal(cache_k[slot // 4, slot % 4], row)
    touched = np.zeros((4, 4), bool)
    touched[[3, 0, 1], [1, 2, 3]] = True
    assert np.array_equal(cache_k[~touched], before[~touched])


def test_slot_indices_known_answers():
    # test_metadata.py:40-57.
    blocks, offsets = slot_indices([0, 5, 2], 4)
    assert blocks.tolist() == [0, 1, 0] and offsets.tolist() == [0, 1, 2]
    blocks, offsets = slot_indices([0, 5, 2], 2)
    assert blocks.tolist() == [0, 2, 1] and offsets.tolist() == [0, 1, 0]
    with pytest.raises(ValueError):
        slot_indices([1], 0)


def test_gather_matches_brute_force_and_handles_empty():
    rng = np.random.default_rng(1)
    cache_k = rng.standard_normal((6, 4, 2, 3)).astype(np.float32)
    cache_v = rng.standard_normal((6, 4, 2, 3)).astype(np.float32)
    tables = [[5, 1, 3], [0, 4, -1], [2, -1, -1]]
    contexts = [9, 0, 4]
    k, v = gather_paged_kv(cache_k, cache_v, tables, contexts, 4)
    expected = [cache_k[tables[r][p // 4], p % 4] for r, c in enumerate(contexts) for p in range(c)]
    np.testing.assert_array_equal(k, np.stack(expected))
    assert v.shape == (13, 2, 3)


def test_decode_slot_construction_known_answer():
    # test_runner.py:57-70: tables [2, 0] and [1] with B = 4, lengths 5 and 2
    # give decode slots [0, 5].
    tables = np.array([[2, 0], [1, -1]], np.int32)
    assert decode_slots(tables, [5, 2], 4).tolist() == [0, 5]


def test_workload_tables_are_disjoint_and_seeded():
    a = make_decode_batch(num_seqs=8, ctx_lo=64, ctx_hi=512, pool_blocks=1024,
                          num_q_heads=16, num_kv_heads=8, head_dim=128, draw_pools=False)
    b = make_decode_batch(num_seqs=8, ctx_lo=64, ctx_hi=512, pool_blocks=1024,
                          num_q_heads=16, num_kv_heads=8, head_dim=128, draw_pools=False)
    assert np.array_equal(a.context_lens, b.context_lens)
    assert np.array_equal(a.block_tables, b.block_tables)
    used = a.block_tables[a.block_tables >= 0]
    assert len(np.unique(used)) == len(used)
    for r, c in enumerate(a.context_lens):
        n = (int(c) + 15) // 16
        assert (a.block_tables[r, :n] >= 0).all() and (a.block_tables[r, n:] == -1).all()
    tables = draw_tables(np.random.default_rng(0), [16, 17], 8, 16)
    assert tables.shape == (2, 2) and tables[0, 1] == -1

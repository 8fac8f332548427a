"""Pins the step-metadata oracle (oracle/step_metadata.py).

Known answers are the reference's own: tests/components/test_runner.py:36-74
(prefill with and without a cached prefix, decode) and
tests/integration/test_cuda_graph.py:62 (bucket list). Random batches are
checked against the closed form of a slot (its block is the table entry of
the position's logical block, its offset the position modulo the block size)
and against decode == one-token prefill at position len-1.
"""

import random

import numpy as np
import pytest

from oracle.step_metadata import decode_rows, graph_buckets, prefill_rows
from tests.support import FakeSeq


def test_prefill_with_prefix_cache_known_answer():
    # test_runner.py:36-50
    a, b = FakeSeq([10, 11, 12, 13, 14, 15]), FakeSeq([24, 25])
    a.num_cached_tokens, a.num_scheduled_tokens, a.block_table = 3, 3, [2, 0]
    b.num_scheduled_tokens, b.block_table = 2, [5]
    m = prefill_rows([a, b], 4)
    assert m["input_ids"].tolist() == [13, 14, 15, 24, 25]
    assert m["positions"].tolist() == [3, 4, 5, 0, 1]
    assert m["cu_seqlens_q"].tolist() == [0, 3, 5]
    assert m["cu_seqlens_k"].tolist() == [0, 6, 8]
    assert (m["max_seqlen_q"], m["max_seqlen_k"]) == (3, 6)
    assert m["slot_mapping"].tolist() == [11, 0, 1, 20, 21]
    assert m["slot_mapping"].dtype == np.int32
    assert m["block_tables"].tolist() == [[2, 0], [5, -1]]


def test_prefill_without_cache_has_no_table():
    # test_runner.py:53-58
    seq = FakeSeq([1, 2])
    seq.num_scheduled_tokens, seq.block_table = 2, [0]
    m = prefill_rows([seq], 4)
    assert m["block_tables"] is None
    assert m["cu_seqlens_k"].tolist() == m["cu_seqlens_q"].tolist() == [0, 2]


def test_decode_known_answer():
    # test_runner.py:61-74
    a, b = FakeSeq([1, 2, 3, 4, 5]), FakeSeq([7, 8])
    a.block_table, b.block_table = [2, 0], [1]
    m = decode_rows([a, b], 4)
    assert m["input_ids"].tolist() == [5, 8]
    assert m["positions"].tolist() == [4, 1]
    assert m["context_lens"].tolist() == [5, 2]
    assert m["slot_mapping"].tolist() == [0, 5]
    assert m["block_tables"].tolist() == [[2, 0], [1, -1]]


def test_invalid_prefill_range_raises():
    seq = FakeSeq([1, 2])
    seq.num_cached_tokens, seq.num_scheduled_tokens, seq.block_table = 2, 1, [0]
    with pytest.raises(ValueError, match="invalid scheduled prefill range"):
        prefill_rows([seq], 4)


def test_graph_bucket_lists():
    assert graph_buckets(4) == [1, 2, 4]  # test_cuda_graph.py:62
    assert graph_buckets(16) == [1, 2, 4, 8, 16]
    assert graph_buckets(40) == [1, 2, 4, 8, 16, 32, 40]
    assert graph_buckets(64) == [1, 2, 4, 8, 16, 32, 48, 64]
    assert graph_buckets(3) == [1, 2, 3]


def random_batch(rng, n, block_size, pool, prefill):
    ids = rng.sample(range(pool), pool)
    seqs, used = [], 0
    for _ in range(n):
        length = rng.randint(1, 6 * block_size)
        seq = FakeSeq([rng.randrange(1000) for _ in range(length)])
        nblk = (length + block_size - 1) // block_size + rng.randint(0, 2)
        seq.block_table = ids[used:used + nblk]
        used += nblk
        if prefill:
            seq.num_cached_tokens = rng.randint(0, length - 1)
            seq.num_scheduled_tokens = rng.randint(1, length - seq.num_cached_tokens)
        seqs.append(seq)
    return seqs


@pytest.mark.parametrize("block_size", [1, 3, 4, 16])
def test_slots_follow_closed_form(block_size):
    rng = random.Random(block_size)
    for n in (1, 5, 12):
        seqs = random_batch(rng, n, block_size, 2000, prefill=True)
        m = prefill_rows(seqs, block_size)
        cu = m["cu_seqlens_q"]
        for r, seq in enumerate(seqs):
            pos = m["positions"][cu[r]:cu[r + 1]]
            slots = m["slot_mapping"][cu[r]:cu[r + 1]].astype(np.int64)
            table = np.asarray(seq.block_table)
            assert (slots // block_size == table[pos // block_size]).all()
            assert (slots % block_size == pos % block_size).all()
            assert pos[0] == seq.num_cached_tokens
            assert (m["input_ids"][cu[r]:cu[r + 1]] == np.asarray(seq.token_ids)[pos]).all()


def test_decode_equals_one_token_prefill_and_pad_rows():
    rng = random.Random(7)
    seqs = random_batch(rng, 9, 16, 500, prefill=False)
    for seq in seqs:
        seq.num_cached_tokens, seq.num_scheduled_tokens = len(seq) - 1, 1
    d = decode_rows(seqs, 16, rows=16, width=40, pad_block=499)
    p = prefill_rows(seqs, 16)
    for key in ("input_ids", "positions", "slot_mapping"):
        assert (d[key][:9] == p[key]).all()
    assert (d["context_lens"][:9] == np.diff(p["cu_seqlens_k"])).all()
    assert (d["block_tables"][:9, :p["block_tables"].shape[1]] == p["block_tables"]).all()
    assert (d["block_tables"][:9, p["block_tables"].shape[1]:] == -1).all()
    # Pad rows: runner.py:567-575.
    assert d["context_lens"][9:].tolist() == [1] * 7
    assert d["slot_mapping"][9:].tolist() == [499 * 16 + i % 16 for i in range(9, 16)]
    assert (d["block_tables"][9:, 0] == 499).all() and (d["block_tables"][9:, 1:] == -1).all()
    assert (d["input_ids"][9:] == 0).all() and (d["positions"][9:] == 0).all()

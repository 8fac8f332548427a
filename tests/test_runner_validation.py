"""Debug-mode step validation (``runner.validate_step``) on the CPU.

Restates the reference's runner debug cases (tests/components/
test_runner.py:120-165): consistent prefill and decode steps pass, duplicate
slots and out-of-range slots/blocks are rejected. Then each invariant of
``ModelRunner.validate_step`` (microinfer/runner.py:387-528) is broken once
in an otherwise consistent step and must raise ValueError with the
reference's message: negative slots, positions at or past ``max_pos_embed``,
token ids outside the vocabulary, non-monotone or inconsistent
``cu_seqlens``, tables that do not cover the tokens, decode rows whose
context, position or slot disagrees with the sequence. The metadata is the
one the oracle (oracle/step_metadata.py) says the device builds, as CPU
tensors.
"""

import numpy as np
import pytest
import torch

from microinfer_amd.layer.metadata import AttentionMetadata
from microinfer_amd.runner import validate_step
from oracle.step_metadata import decode_rows, prefill_rows
from tests.support import FakeSeq

B = 4


def seq(tokens, cached=0, scheduled=None, table=()):
    s = FakeSeq(tokens)
    s.num_cached_tokens = cached
    s.num_scheduled_tokens = len(tokens) - cached if scheduled is None else scheduled
    s.block_table = list(table)
    return s


def prefill_step(seqs, **edit):
    rows = prefill_rows(seqs, B)
    rows.update(edit)
    t = lambda a: None if a is None else torch.as_tensor(np.asarray(a))  # noqa: E731
    meta = AttentionMetadata.build(
        is_prefill=True, cu_seqlens_q=t(rows["cu_seqlens_q"]),
        cu_seqlens_k=t(rows["cu_seqlens_k"]), max_seqlen_q=rows["max_seqlen_q"],
        max_seqlen_k=rows["max_seqlen_k"], slot_mapping=t(rows["slot_mapping"]),
        block_tables=t(rows["block_tables"]), validate_cache_write=True)
    return t(rows["input_ids"]), t(rows["positions"]), meta


def decode_step(seqs, **edit):
    rows = decode_rows(seqs, B)
    rows.update(edit)
    t = lambda a: torch.as_tensor(np.asarray(a))  # noqa: E731
    meta = AttentionMetadata.build(
        is_prefill=False, slot_mapping=t(rows["slot_mapping"]),
        context_lens=t(rows["context_lens"]), block_tables=t(rows["block_tables"]),
        validate_cache_write=True)
    return t(rows["input_ids"]), t(rows["positions"]), meta


def check(seqs, step, is_prefill, **limits):
    validate_step(seqs, *step, is_prefill, block_size=B, **limits)


def test_consistent_prefill_and_decode_pass():
    # test_runner.py:120-137.
    s = seq([1, 2, 3, 4], table=[0])
    check([s], prefill_step([s]), True, num_blocks=1, max_pos_embed=8, vocab_size=8)
    d = seq([1, 2, 3, 4, 5], cached=4, scheduled=1, table=[0, 1])
    check([d], decode_step([d]), False, num_blocks=2, max_pos_embed=8, vocab_size=8)
    # A prefix-cached chunk with a table, beside a fresh one.
    a, b = seq([5, 6, 7, 8, 9, 10], cached=3, table=[2, 0]), seq([3, 4], table=[5])
    check([a, b], prefill_step([a, b]), True, num_blocks=6)


def test_duplicate_slots_rejected():
    # test_runner.py:140-146: two sequences sharing block 0.
    a, b = seq([1, 2], table=[0]), seq([3, 4], table=[0])
    with pytest.raises(ValueError, match="duplicate"):
        check([a, b], prefill_step([a, b]), True)


def test_out_of_range_slot_rejected():
    # test_runner.py:157-170: block 99 in a 2-block pool.
    s = seq([1, 2, 3, 4, 5], cached=1, scheduled=3, table=[99])
    with pytest.raises(ValueError, match="KV capacity|block"):
        check([s], prefill_step([s]), True, num_blocks=2)


PREFILL_BREAKS = {
    "negative slot": (dict(slot_mapping=[-1, 1, 2]), "nonnegative"),
    "position past max_pos_embed": ({}, "max_pos_embed"),
    "token outside vocabulary": (dict(input_ids=[1, 2, 99]), "vocabulary"),
    "cu_seqlens_q non-monotone": (dict(cu_seqlens_q=[0, 4, 3]), "query length|endpoints"),
    "cu_seqlens_k wrong": (dict(cu_seqlens_k=[0, 2, 5]), "KV length"),
    "max_seqlen_q wrong": (dict(max_seqlen_q=7), "max_seqlen_q"),
    "positions shifted": (dict(positions=[1, 2, 3]), "positions do not match"),
    "slots off the table": (dict(slot_mapping=[4, 1, 2]), "slot_mapping does not match"),
}


@pytest.mark.parametrize("case", sorted(PREFILL_BREAKS))
def test_prefill_invariants(case):
    edit, message = PREFILL_BREAKS[case]
    a, b = seq([1, 2], table=[0]), seq([3], table=[1])
    limits = dict(num_blocks=2, vocab_size=8,
                  max_pos_embed=1 if case == "position past max_pos_embed" else 8)
    with pytest.raises(ValueError, match=message):
        check([a, b], prefill_step([a, b], **edit), True, **limits)


def test_uncovered_tables_rejected():
    s = seq([1, 2, 3, 4, 5, 6], table=[0])  # 6 tokens need 2 blocks of 4
    with pytest.raises(ValueError, match="cover"):
        validate_step([s], torch.tensor([1, 2, 3, 4, 5, 6]), torch.arange(6),
                      AttentionMetadata.build(
                          is_prefill=True, cu_seqlens_q=torch.tensor([0, 6]),
                          cu_seqlens_k=torch.tensor([0, 6]), max_seqlen_q=6, max_seqlen_k=6,
                          slot_mapping=torch.tensor([0, 1, 2, 3, 4, 5]), block_tables=None,
                          validate_cache_write=True),
                      True, block_size=B)
    d = seq([1, 2, 3, 4, 5], cached=4, scheduled=1, table=[0, 1])
    ids, pos, meta = decode_step([d])
    meta = AttentionMetadata.build(is_prefill=False, slot_mapping=meta.slot_mapping,
                                   context_lens=meta.context_lens,
                                   block_tables=torch.tensor([[0, -1]], dtype=torch.int32),
                                   validate_cache_write=True)
    with pytest.raises(ValueError, match="negative block id|cover"):
        validate_step([d], ids, pos, meta, False, block_size=B)


DECODE_BREAKS = {
    "context length": (dict(context_lens=[4, 2]), "context length"),
    "position": (dict(positions=[3, 1]), "decode position"),
    "slot": (dict(slot_mapping=[5, 5]), "duplicate|decode slot"),
    "block past pool": (dict(block_tables=[[0, 1], [7, -1]]), "KV pool|KV capacity"),
}


@pytest.mark.parametrize("case", sorted(DECODE_BREAKS))
def test_decode_invariants(case):
    edit, message = DECODE_BREAKS[case]
    a = seq([1, 2, 3, 4, 5], cached=4, scheduled=1, table=[0, 1])
    b = seq([6, 7], cached=1, scheduled=1, table=[2])
    check([a, b], decode_step([a, b]), False, num_blocks=3)  # consistent as built
    with pytest.raises(ValueError, match=message):
        check([a, b], decode_step([a, b], **edit), False, num_blocks=3)


def test_mode_and_shape_checks():
    s = seq([1, 2], table=[0])
    ids, pos, meta = prefill_step([s])
    with pytest.raises(ValueError, match="mode"):
        validate_step([s], ids, pos, meta, False, block_size=B)
    with pytest.raises(ValueError, match="requests"):
        validate_step([], ids, pos, meta, True, block_size=B)
    with pytest.raises(ValueError, match="equal length"):
        validate_step([s], ids, pos[:1], meta, True, block_size=B)

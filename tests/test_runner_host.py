"""Host side of the device metadata build (microinfer_amd/runner.py), no GPU.

The bucket list must equal the oracle's restatement of runner.py:275-283;
scheduler contract violations raise ValueError before anything is sent to the
device; a valid batch on a CPU device raises RuntimeError (there is no CPU
fallback); the C entry rejects bad sizes without launching. The host packing
(description layout, pointers, column bookkeeping) is checked by replacing the
launch with a numpy emulation of mi_step_metadata as include/mi_attn.h
specifies it and comparing every output with the oracle.
"""

import ctypes
import random

import numpy as np
import pytest

from microinfer_amd import _lib
from microinfer_amd.runner import DecodeBuffers, StepMetadataBuilder, graph_buckets
from oracle.step_metadata import decode_rows, prefill_rows
from oracle.step_metadata import graph_buckets as oracle_buckets
from tests.support import FakeSeq
from tests.test_oracle_step_metadata import random_batch


def test_bucket_list_matches_oracle():
    for m in range(1, 300):
        assert graph_buckets(m) == oracle_buckets(m)
    with pytest.raises(ValueError):
        graph_buckets(0)


def _seq(tokens, cached, scheduled, table):
    s = FakeSeq(tokens)
    s.num_cached_tokens, s.num_scheduled_tokens, s.block_table = cached, scheduled, table
    return s


def test_prefill_contract_errors_come_first():
    b = StepMetadataBuilder(4, "cpu")
    with pytest.raises(ValueError, match="invalid scheduled prefill range"):
        b.prepare_prefill([_seq([1, 2], 2, 1, [0])])
    with pytest.raises(ValueError, match="invalid scheduled prefill range"):
        b.prepare_prefill([_seq([1, 2], 0, 0, [0])])
    with pytest.raises(ValueError, match="does not cover"):
        b.prepare_prefill([_seq([1, 2, 3, 4, 5], 0, 5, [0])])
    with pytest.raises(ValueError, match="int32"):
        b.prepare_prefill([_seq([1, 2], 0, 2, [2 ** 30])])
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        b.prepare_prefill([_seq([1, 2], 0, 2, [0])])


def test_decode_contract_errors_come_first():
    b = StepMetadataBuilder(4, "cpu")
    with pytest.raises(ValueError, match="does not cover"):
        b.prepare_decode([_seq([1, 2, 3, 4, 5], 4, 1, [7])])
    buffers = DecodeBuffers("cpu", 2, 2)
    with pytest.raises(ValueError, match="pad block"):
        b.fill_decode(buffers, [_seq([1], 0, 1, [0])], rows=2)
    with pytest.raises(ValueError, match="wider"):
        b.fill_decode(buffers, [_seq([1], 0, 1, [0, 1, 2])])
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        b.prepare_decode([_seq([1, 2], 1, 1, [3])])


def test_empty_batches_return_empty_tensors():
    b = StepMetadataBuilder(4, "cpu")
    ids, positions, metadata = b.prepare_decode([])
    assert ids.numel() == positions.numel() == 0 and metadata.is_decode
    ids, positions, metadata = b.prepare_prefill([])
    assert ids.numel() == 0 and metadata.is_prefill and metadata.block_tables is None


def test_c_entry_validates_before_launch():
    lib = _lib.load()
    # rows below num_seqs
    assert lib.mi_step_metadata(None, None, None, None, None, 3, 2, 3, 16, -1, None, 0, 0,
                                None, None, None, None, None) == 1
    assert "sizes" in _lib.last_error()
    # pad rows without a pad block
    assert lib.mi_step_metadata(None, None, None, None, None, 1, 2, 2, 16, -1, None, 0, 0,
                                None, None, None, None, None) == 1
    assert "pad block" in _lib.last_error()
    # pad slot beyond int32
    assert lib.mi_step_metadata(None, None, None, None, None, 0, 1, 1, 16, 2 ** 28, None, 0, 0,
                                None, None, None, None, None) == 1
    assert "int32" in _lib.last_error()
    # no rows: nothing to do
    assert lib.mi_step_metadata(None, None, None, None, None, 0, 0, 0, 16, -1, None, 0, 0,
                                None, None, None, None, None) == 0


def _view(ptr, count, ctype):
    if count <= 0:
        return np.zeros(0, dtype=np.int64)
    return np.ctypeslib.as_array((ctype * count).from_address(ptr))


def emulate_step_metadata(_self, args):
    """mi_step_metadata as the header documents it, on host pointers."""
    (cu_q, starts, offsets, blocks, tokens, num_seqs, rows, num_tokens, block_size, pad,
     tables, stride, width, ctx, slots, positions, ids) = args
    i32, i64 = ctypes.c_int32, ctypes.c_int64
    cu = _view(cu_q, num_seqs + 1, i32)
    st = _view(starts, num_seqs, i32)
    off = _view(offsets, num_seqs + 1, i32)
    blk = _view(blocks, int(off[-1]) if num_seqs else 0, i32)
    tok = _view(tokens, int(cu[-1]), i64)
    out_pos, out_ids = _view(positions, num_tokens, i64), _view(ids, num_tokens, i64)
    out_slots = _view(slots, num_tokens, i32)
    out_ctx = _view(ctx, rows, i32) if ctx else None
    for r in range(rows):
        if r < num_seqs:
            t0, count, start = int(cu[r]), int(cu[r + 1] - cu[r]), int(st[r])
            own = blk[off[r]:off[r + 1]]
        else:
            t0, count, start, own = int(cu[num_seqs]) + r - num_seqs, 1, 0, None
        if tables:
            row = _view(tables + 4 * r * stride, width, i32)
            row[:] = -1
            if own is None:
                row[0] = pad
            else:
                row[:min(len(own), width)] = own[:width]
        if out_ctx is not None:
            out_ctx[r] = 1 if own is None else start + count
        for i in range(count):
            t, p = t0 + i, start + i
            out_pos[t] = p
            out_ids[t] = 0 if own is None else tok[t]
            if own is None:
                out_slots[t] = pad * block_size + r % block_size
            else:
                lb = p // block_size
                out_slots[t] = own[lb] * block_size + p % block_size if lb < len(own) else -1


@pytest.fixture
def emulated(monkeypatch):
    monkeypatch.setattr(StepMetadataBuilder, "_run", emulate_step_metadata)


@pytest.mark.parametrize("block_size", [1, 4, 16])
def test_prefill_packing_matches_oracle(emulated, block_size):
    rng = random.Random(block_size)
    b = StepMetadataBuilder(block_size, "cpu")
    for n in (1, 3, 20):
        seqs = random_batch(rng, n, block_size, 3000, prefill=True)
        ids, positions, m = b.prepare_prefill(seqs)
        want = prefill_rows(seqs, block_size)
        assert ids.tolist() == want["input_ids"].tolist()
        assert positions.tolist() == want["positions"].tolist()
        assert m.slot_mapping.tolist() == want["slot_mapping"].tolist()
        assert m.cu_seqlens_q.tolist() == want["cu_seqlens_q"].tolist()
        assert m.cu_seqlens_k.tolist() == want["cu_seqlens_k"].tolist()
        assert (m.max_seqlen_q, m.max_seqlen_k) == (want["max_seqlen_q"], want["max_seqlen_k"])
        if want["block_tables"] is None:
            assert m.block_tables is None
        else:
            assert m.block_tables.tolist() == want["block_tables"].tolist()


def test_decode_packing_and_column_bookkeeping(emulated):
    rng = random.Random(3)
    b = StepMetadataBuilder(4, "cpu", pad_block_id=999)
    for n in (7, 30, 2, 64, 1):  # eager buffers grow and shrink
        seqs = random_batch(rng, n, 4, 3000, prefill=False)
        ids, positions, m = b.prepare_decode(seqs)
        want = decode_rows(seqs, 4, width=m.block_tables.shape[1])
        for got, key in ((ids, "input_ids"), (positions, "positions"),
                         (m.slot_mapping, "slot_mapping"), (m.context_lens, "context_lens"),
                         (m.block_tables, "block_tables")):
            assert got.tolist() == want[key].tolist(), key
    buffers = b.pad_buffers(16, 300)
    for n in (16, 3, 0, 9):  # graph bucket: full rewrite of shrinking tables
        seqs = random_batch(rng, n, 4, 3000, prefill=False)
        b.fill_decode(buffers, seqs, rows=16)
        want = decode_rows(seqs, 4, rows=16, width=300, pad_block=999)
        for key in want:
            assert getattr(buffers, key).tolist() == want[key].tolist(), (n, key)

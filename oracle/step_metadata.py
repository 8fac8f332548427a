"""numpy restatement of MicroInfer's per-step metadata build (test infrastructure).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this module. It is what results are compared with, never the thing measured or
shipped.

A scheduled sequence is any object with ``len()``, indexing over its token
ids, ``last_token``, ``block_table`` (list of physical block ids),
``num_cached_tokens`` and ``num_scheduled_tokens`` -- the attributes
``ModelRunner`` reads from ``microinfer/engine/sequence.py:14-45``.

How each function is pinned (tests/test_oracle_step_metadata.py):

* ``prefill_rows`` -- the reference's known answers
  (tests/components/test_runner.py:36-50: prefix-cached prefill of two
  sequences at B=4 -> ids [13,14,15,24,25], positions [3,4,5,0,1],
  cu_q [0,3,5], cu_k [0,6,8], max (3,6), slots [11,0,1,20,21], tables
  [[2,0],[5,-1]]; :53-58 no cached tokens -> no table, cu_k == cu_q), and the
  closed form ``slot // B == table[pos // B]``, ``slot % B == pos % B`` over
  random batches.
* ``decode_rows`` -- test_runner.py:61-74 (ids [5,8], positions [4,1],
  context [5,2], slots [0,5], tables [[2,0],[1,-1]]); it must equal
  ``prefill_rows`` for the same sequences scheduled as one-token chunks at
  position len-1; pad rows follow runner.py:203-215 / :567-575 (ctx 1,
  slot pad*B + i % B, table [pad, -1, ...]).
* ``graph_buckets`` -- tests/integration/test_cuda_graph.py:62 (max 4 ->
  [1, 2, 4]) and the list rule of runner.py:275-283.
"""

from __future__ import annotations

import numpy as np


def graph_buckets(max_num_seqs: int) -> list[int]:
    """Decode batch sizes captured as graphs (microinfer/runner.py:275-283)."""
    buckets = [1, 2, 4, 8] + list(range(16, max_num_seqs + 1, 16))
    buckets = sorted({b for b in buckets if b <= max_num_seqs})
    if not buckets:
        buckets = [1]
    if buckets[-1] != max_num_seqs:
        buckets.append(max_num_seqs)
    return buckets


def _slot(block_table, position: int, block_size: int) -> int:
    # runner.py:169-172 (decode) and :313-317 (prefill).
    return block_table[position // block_size] * block_size + position % block_size


def decode_rows(seqs, block_size: int, *, rows: int | None = None, width: int | None = None,
                pad_block: int | None = None):
    """Decode-step metadata as ``ModelRunner`` fills it.

    Follows ``_fill_decode_rows`` (microinfer/runner.py:160-176): one row per
    sequence with ``input_ids = last_token``, ``positions = len - 1``,
    ``slot_mapping = table[p // B] * B + p % B``, ``context_lens = len`` and
    the block table padded with -1. ``rows > len(seqs)`` adds the graph pad
    rows of ``_fill_graph_bucket`` (:561-576): ids 0, positions 0, context 1,
    slot ``pad_block * B + i % B`` and table ``[pad_block, -1, ...]``.
    ``width`` defaults to the longest table (``prepare_decode``, :349).
    """
    batch = len(seqs)
    rows = batch if rows is None else rows
    if rows < batch:
        raise ValueError("rows must cover every sequence")
    if rows > batch and pad_block is None:
        raise ValueError("pad rows need a pad block")
    if width is None:
        width = max((len(s.block_table) for s in seqs), default=0)
        if rows > batch:
            width = max(width, 1)
    out = {
        "input_ids": np.zeros(rows, dtype=np.int64),
        "positions": np.zeros(rows, dtype=np.int64),
        "slot_mapping": np.zeros(rows, dtype=np.int32),
        "context_lens": np.zeros(rows, dtype=np.int32),
        "block_tables": np.full((rows, width), -1, dtype=np.int32),
    }
    for i, seq in enumerate(seqs):
        position = len(seq) - 1
        out["input_ids"][i] = seq.last_token
        out["positions"][i] = position
        out["slot_mapping"][i] = _slot(seq.block_table, position, block_size)
        out["context_lens"][i] = len(seq)
        out["block_tables"][i, :len(seq.block_table)] = seq.block_table
    for i in range(batch, rows):
        out["context_lens"][i] = 1
        out["slot_mapping"][i] = pad_block * block_size + i % block_size
        out["block_tables"][i, 0] = pad_block
    return out


def prefill_rows(seqs, block_size: int):
    """Prefill-step metadata as ``ModelRunner.prepare_prefill`` builds it.

    Follows microinfer/runner.py:298-346: sequence ``s`` schedules positions
    ``[num_cached, num_cached + num_scheduled)``; ``cu_seqlens_q`` sums the
    scheduled counts, ``cu_seqlens_k`` the end positions; the block table
    (``prepare_block_tables``, :290-296, -1 padded to the longest table) is
    only built when some sequence has cached tokens.
    """
    ids, positions, slots, cu_q, cu_k = [], [], [], [0], [0]
    for seq in seqs:
        start = seq.num_cached_tokens
        end = start + seq.num_scheduled_tokens
        if not 0 <= start < end <= len(seq):
            raise ValueError("invalid scheduled prefill range")
        ids.extend(seq[start:end])
        positions.extend(range(start, end))
        cu_q.append(cu_q[-1] + end - start)
        cu_k.append(cu_k[-1] + end)
        slots.extend(_slot(seq.block_table, p, block_size) for p in range(start, end))
    tables = None
    if any(s.num_cached_tokens for s in seqs):
        width = max((len(s.block_table) for s in seqs), default=0)
        tables = np.full((len(seqs), width), -1, dtype=np.int32)
        for i, seq in enumerate(seqs):
            tables[i, :len(seq.block_table)] = seq.block_table
    return {
        "input_ids": np.asarray(ids, dtype=np.int64),
        "positions": np.asarray(positions, dtype=np.int64),
        "slot_mapping": np.asarray(slots, dtype=np.int32),
        "cu_seqlens_q": np.asarray(cu_q, dtype=np.int32),
        "cu_seqlens_k": np.asarray(cu_k, dtype=np.int32),
        "max_seqlen_q": max((s.num_scheduled_tokens for s in seqs), default=0),
        "max_seqlen_k": max((s.num_cached_tokens + s.num_scheduled_tokens for s in seqs),
                            default=0),
        "block_tables": tables,
    }

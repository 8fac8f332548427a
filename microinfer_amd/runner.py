"""Per-step attention metadata built on the device, and graph-captured decode.

Mirrors the metadata half of ``ModelRunner`` (microinfer/runner.py):
``prepare_prefill`` (:298-346), ``prepare_decode`` (:348-385),
``prepare_block_tables`` (:290-296), the decode buffers of ``_DecodeBuffers``
(:16-48), the graph buckets of ``capture_cuda_graphs`` (:275-283), the pad
rows of ``_fill_pad_buffers`` / ``_fill_graph_bucket`` (:203-215, :561-576)
and the bucket capture and replay of ``_capture_bucket`` / ``_run_decode``
(:217-250, :578-604).

The reference fills every row in Python and copies full-width tables to the
device each step (``[bucket, num_blocks + 1]`` int32 for a graph bucket).
Here the host packs only what the scheduler decided -- each sequence's first
scheduled position, its token count, the block ids it owns and the scheduled
token ids -- into a pinned buffer, sends it with one asynchronous copy, and
``mi_step_metadata`` expands it on the device into the int32/int64 tensors the
attention kernels and the model read.

A scheduled sequence is any object with ``len()``, slicing over its token ids,
``last_token``, ``block_table``, ``num_cached_tokens`` and
``num_scheduled_tokens`` (``microinfer/engine/sequence.py:14-45``).
"""

from __future__ import annotations

import contextlib
import gc
from itertools import chain

import numpy as np
import torch

from microinfer_amd import _lib
from microinfer_amd.layer.hip_sampler import greedy_argmax
from microinfer_amd.layer.metadata import AttentionMetadata

_INT32_MAX = 2 ** 31 - 1


@contextlib.contextmanager
def capture_graph(graph, pool=None, stream=None):
    """``torch.cuda.graph(graph, pool, stream=stream)`` with Python's cyclic
    garbage collector kept off for the whole capture.

    Objects that hold graphs (a runner whose graph runner calls back into it
    forms a reference cycle) are freed only by that collector; if it ran
    during a capture, destroying such a graph would be a HIP call that is
    illegal while a stream captures, and the process would abort. So collect
    what is already garbage first, then capture with the collector disabled
    (torch's own capture no longer collects by default)."""
    gc.collect()
    enabled = gc.isenabled()
    gc.disable()
    try:
        with torch.cuda.graph(graph, pool, stream=stream):
            yield
    finally:
        if enabled:
            gc.enable()


def graph_buckets(max_num_seqs: int) -> list[int]:
    """Decode batch sizes captured as graphs: 1, 2, 4, 8, multiples of 16 and
    ``max_num_seqs`` itself (microinfer/runner.py:275-283)."""
    if max_num_seqs < 1:
        raise ValueError("max_num_seqs must be positive")
    buckets = sorted({b for b in [1, 2, 4, 8, *range(16, max_num_seqs + 1, 16)]
                      if b <= max_num_seqs})
    if buckets[-1] != max_num_seqs:
        buckets.append(max_num_seqs)
    return buckets


def _host_ints(tensor) -> list[int]:
    return [int(v) for v in tensor.reshape(-1).tolist()]


def validate_step(seqs, input_ids, positions, metadata, is_prefill: bool, *, block_size: int,
                  num_blocks: int | None = None, max_pos_embed: int | None = None,
                  vocab_size: int | None = None) -> None:
    """Debug-mode check of one step's metadata against the scheduled sequences.

    Restates ``ModelRunner.validate_step`` (microinfer/runner.py:387-528):
    the same invariants, raised as ValueError with the reference's messages,
    before anything is launched. The device-built tensors are read back once
    (a synchronising copy), which is why this runs only in debug mode.
    ``num_blocks`` is the pool the scheduler hands out, ``max_pos_embed`` and
    ``vocab_size`` the model's limits (each check is skipped when None).
    """
    if metadata.is_prefill is not is_prefill:
        raise ValueError("metadata mode does not match scheduled work")
    if input_ids.ndim != 1 or positions.ndim != 1:
        raise ValueError("input_ids and positions must be 1-D")
    if input_ids.numel() != positions.numel() or input_ids.numel() == 0:
        raise ValueError("input_ids/positions must be nonempty and equal length")
    if not seqs:
        raise ValueError("a scheduled batch must contain requests")
    slots = metadata.slot_mapping
    if slots is None or slots.ndim != 1 or slots.numel() != input_ids.numel():
        raise ValueError("slot_mapping must match scheduled tokens")
    slot_list, pos_list, id_list = _host_ints(slots), _host_ints(positions), _host_ints(input_ids)
    if min(slot_list) < 0:
        raise ValueError("slot_mapping must be nonnegative")
    if len(set(slot_list)) != len(slot_list):
        raise ValueError("slot_mapping contains duplicate slots")
    if num_blocks is not None and max(slot_list) >= num_blocks * block_size:
        raise ValueError("slot_mapping exceeds KV capacity")
    if min(pos_list) < 0:
        raise ValueError("positions must be nonnegative")
    if max_pos_embed is not None and max(pos_list) >= max_pos_embed:
        raise ValueError("position exceeds model max_pos_embed")
    if min(id_list) < 0:
        raise ValueError("input_ids must be nonnegative")
    if vocab_size is not None and max(id_list) >= vocab_size:
        raise ValueError("input_ids exceed model vocabulary")

    def covered(ids, needed: int, short_message: str) -> None:
        if len(ids) < needed:
            raise ValueError(short_message)
        for block_id in ids[:needed]:
            if int(block_id) < 0:
                raise ValueError("block table contains a negative block id")
            if num_blocks is not None and int(block_id) >= num_blocks:
                raise ValueError("block id exceeds KV pool")

    def slot_of(seq, position: int) -> int:
        return int(seq.block_table[position // block_size]) * block_size + position % block_size

    # Per request: the context the step's attention reads (cached + scheduled
    # tokens for prefill, the whole sequence for decode).
    contexts = []
    if is_prefill:
        if metadata.cu_seqlens_q is None or metadata.cu_seqlens_k is None:
            raise ValueError("prefill requires cu_seqlens_q/cu_seqlens_k")
        cu_q, cu_k = _host_ints(metadata.cu_seqlens_q), _host_ints(metadata.cu_seqlens_k)
        if len(cu_q) != len(seqs) + 1 or len(cu_k) != len(seqs) + 1:
            raise ValueError("cu_seqlens must contain num_requests + 1 entries")
        if cu_q[0] != 0 or cu_k[0] != 0 or cu_q[-1] != input_ids.numel():
            raise ValueError("invalid cu_seqlens endpoints")
        q_lens = [b - a for a, b in zip(cu_q, cu_q[1:])]
        k_lens = [b - a for a, b in zip(cu_k, cu_k[1:])]
        for i, seq in enumerate(seqs):
            start = seq.num_cached_tokens
            end = start + seq.num_scheduled_tokens
            if q_lens[i] <= 0:
                raise ValueError("prefill query length must be positive")
            if q_lens[i] != seq.num_scheduled_tokens:
                raise ValueError("query length does not match scheduled tokens")
            if k_lens[i] != end:
                raise ValueError("KV length does not match cached+scheduled tokens")
            if len(seq) < end:
                raise ValueError("scheduled tokens exceed sequence length")
            covered(seq.block_table, -(-end // block_size),
                    "block table does not cover scheduled tokens")
            if pos_list[cu_q[i]:cu_q[i + 1]] != list(range(start, end)):
                raise ValueError("positions do not match prefill range")
            if slot_list[cu_q[i]:cu_q[i + 1]] != [slot_of(seq, p) for p in range(start, end)]:
                raise ValueError("slot_mapping does not match block table")
            contexts.append(end)
        if cu_q[-1] != sum(q_lens) or cu_k[-1] != sum(k_lens):
            raise ValueError("cu_seqlens totals do not match")
        if metadata.max_seqlen_q != max(q_lens):
            raise ValueError("max_seqlen_q does not match cu_seqlens_q")
        if metadata.max_seqlen_k != max(k_lens):
            raise ValueError("max_seqlen_k does not match cu_seqlens_k")
        if any(seq.num_cached_tokens for seq in seqs) and metadata.block_tables is None:
            raise ValueError("cached prefixes require block_tables")
    else:
        if len(seqs) != input_ids.numel():
            raise ValueError("decode needs exactly one token per request")
        if metadata.context_lens is None or metadata.context_lens.numel() != len(seqs):
            raise ValueError("decode requires one context length per request")
        if metadata.block_tables is None:
            raise ValueError("decode requires block_tables")
        for i, (seq, context) in enumerate(zip(seqs, _host_ints(metadata.context_lens))):
            if context != len(seq) or context <= 0:
                raise ValueError("context length does not match sequence length")
            if pos_list[i] != context - 1:
                raise ValueError("decode position does not match context length")
            covered(seq.block_table, -(-context // block_size),
                    "block table does not cover scheduled tokens")
            if slot_list[i] != slot_of(seq, context - 1):
                raise ValueError("decode slot does not match block table")
            contexts.append(context)
    tables = metadata.block_tables
    if tables is not None:
        if tables.ndim != 2 or tables.shape[0] != len(seqs):
            raise ValueError("block_tables must be [num_requests, max_blocks]")
        for row, context in zip(tables.tolist(), contexts):
            covered(row, -(-context // block_size), "block table does not cover context")


class DecodeBuffers:
    """Device tensors a decode step writes its metadata into.

    Same names and dtypes as ``_DecodeBuffers`` (microinfer/runner.py:8-48):
    int64 ``input_ids`` / ``positions``, int32 ``slot_mapping`` /
    ``context_lens`` and an int32 ``block_tables [capacity, width]``. There is
    no host mirror: the rows are written on the device.
    """

    def __init__(self, device, capacity: int = 0, width: int = 0):
        self.device = torch.device(device)
        self.capacity = -1
        self.width = -1
        self.ensure(capacity, width)

    def ensure(self, batch: int, width: int) -> None:
        if batch <= self.capacity and width <= self.width:
            return
        capacity, width = max(batch, self.capacity, 0), max(width, self.width, 0)
        dev = self.device
        self.input_ids = torch.empty(capacity, dtype=torch.int64, device=dev)
        self.positions = torch.empty(capacity, dtype=torch.int64, device=dev)
        self.slot_mapping = torch.empty(capacity, dtype=torch.int32, device=dev)
        self.context_lens = torch.empty(capacity, dtype=torch.int32, device=dev)
        self.block_tables = torch.empty((capacity, width), dtype=torch.int32, device=dev)
        self.capacity, self.width = capacity, width
        # Columns at or past this index are -1 in every row (a new table holds
        # garbage everywhere).
        self.table_written = width

    def metadata(self, batch: int) -> AttentionMetadata:
        """Decode metadata over the first ``batch`` rows (``_make_decode_metadata``,
        microinfer/runner.py:190-197)."""
        return AttentionMetadata.build(
            is_prefill=False,
            slot_mapping=self.slot_mapping[:batch],
            context_lens=self.context_lens[:batch],
            block_tables=self.block_tables[:batch],
            validate_cache_write=False,
        )


class _Upload:
    """Two pinned host buffers, used in turn, for the compact step description.

    Before a buffer is rewritten the host waits for the copy that last read
    it, so the host can run one step ahead of the device without racing its
    own uploads. A description is int64 token ids followed by int32 arrays.
    """

    def __init__(self, device: torch.device):
        self.device = device
        self.pinned = device.type == "cuda"
        self._slots = [None, None]  # [host tensor, int64 view, int32 view, event]
        self._turn = 0
        self._staged = None

    def stage(self, words: int):
        """(int64, int32) numpy views of a host buffer of at least ``words``
        int64 words that no pending copy still reads."""
        i = self._turn
        self._turn ^= 1
        slot = self._slots[i]
        if slot is None or slot[0].numel() < words:
            size = max(words, 4096, 0 if slot is None else 2 * slot[0].numel())
            host = torch.empty(size, dtype=torch.int64, pin_memory=self.pinned)
            slot = [host, host.numpy(), host.view(torch.int32).numpy(), None]
            self._slots[i] = slot
        elif slot[3] is not None:
            slot[3].synchronize()
        self._staged = slot
        return slot[1], slot[2]

    def commit(self, dst: torch.Tensor, words: int) -> None:
        """Copy the first ``words`` staged words into the int64 device tensor
        ``dst``, asynchronously on the current stream."""
        slot = self._staged
        dst[:words].copy_(slot[0][:words], non_blocking=self.pinned)
        if self.pinned:
            if slot[3] is None:
                slot[3] = torch.cuda.Event()
            slot[3].record(torch.cuda.current_stream(self.device))


class StepMetadataBuilder:
    """Builds each step's ``(input_ids, positions, AttentionMetadata)`` on the device.

    ``pad_block_id`` is the block a graph runner reserves past the scheduler's
    pool for pad rows (``allocate_kv_cache``, microinfer/runner.py:134-153);
    it is only needed for graph buckets.

    With ``debug_mode`` every step is checked by ``validate_step`` before it
    is returned (and so before anything reads it), against ``num_blocks``,
    ``max_pos_embed`` and ``vocab_size`` where given, and the metadata asks
    for checked cache writes, as the reference's debug mode does
    (microinfer/runner.py:337-346, :378-384).
    """

    def __init__(self, block_size: int, device, *, pad_block_id: int | None = None,
                 debug_mode: bool = False, num_blocks: int | None = None,
                 max_pos_embed: int | None = None, vocab_size: int | None = None):
        if block_size <= 0:
            raise ValueError("block_size must be positive")
        self.block_size = block_size
        self.device = torch.device(device)
        self.pad_block_id = pad_block_id
        self.debug_mode = debug_mode
        self.limits = dict(block_size=block_size, num_blocks=num_blocks,
                           max_pos_embed=max_pos_embed, vocab_size=vocab_size)
        self._upload = _Upload(self.device)
        self._decode_buffers: DecodeBuffers | None = None
        self._decode_upload: torch.Tensor | None = None

    def _check_blocks(self, last_positions: np.ndarray, counts: np.ndarray,
                      blocks: np.ndarray) -> None:
        """Every table covers its last scheduled position; every slot fits int32."""
        if last_positions.size and (last_positions // self.block_size >= counts).any():
            raise ValueError("block table does not cover scheduled tokens")
        if blocks.size and int(blocks.max()) * self.block_size + self.block_size - 1 > _INT32_MAX:
            raise ValueError("slot ids exceed int32")

    def _launch(self, base: int, n_tok: int, layout, num_seqs, rows, num_tokens, tables,
                table_stride, width, context_lens, slots, positions, input_ids):
        """``layout`` = int32 word offsets (after the tokens) of cu_q, starts,
        block offsets and blocks in the uploaded description at ``base``."""
        at = base + 8 * n_tok
        cu_q, starts, offsets, blocks = (at + 4 * w for w in layout)
        self._run((cu_q, starts, offsets, blocks, base, num_seqs, rows, num_tokens,
                   self.block_size, -1 if self.pad_block_id is None else self.pad_block_id,
                   tables, table_stride, width, context_lens, slots, positions, input_ids))

    def _run(self, args) -> None:
        """Call ``mi_step_metadata`` with ``args`` (all but the stream)."""
        if self.device.type != "cuda":
            raise RuntimeError("mi_step_metadata needs a HIP device (no CPU fallback)")
        status = _lib.load().mi_step_metadata(*args, _lib.stream_handle(self.device))
        _lib.check(status, "mi_step_metadata")

    # -- prefill --------------------------------------------------------------
    def prepare_prefill(self, seqs):
        """``ModelRunner.prepare_prefill`` (microinfer/runner.py:298-346) on the device."""
        n = len(seqs)
        starts = np.array([s.num_cached_tokens for s in seqs], dtype=np.int64)
        counts = np.array([s.num_scheduled_tokens for s in seqs], dtype=np.int64)
        lengths = np.array([len(s) for s in seqs], dtype=np.int64)
        ends = starts + counts
        if n and ((starts < 0) | (ends <= starts) | (ends > lengths)).any():
            raise ValueError("invalid scheduled prefill range")
        if n and max(int(ends.sum()), int(counts.sum())) > _INT32_MAX:
            raise ValueError("scheduled tokens exceed int32")
        tables = [s.block_table for s in seqs]
        t_counts = np.array([len(t) for t in tables], dtype=np.int64)
        flat = np.array(list(chain.from_iterable(tables)), dtype=np.int64)
        self._check_blocks(ends - 1, t_counts, flat)
        total = int(counts.sum())
        tokens = list(chain.from_iterable(s[a:b] for s, a, b in zip(seqs, starts.tolist(),
                                                                       ends.tolist())))
        with_tables = bool((starts > 0).any())
        width = int(t_counts.max()) if (with_tables and n) else 0

        # int32 words after the tokens: cu_q | cu_k | starts | block offsets | blocks.
        n32 = 4 * n + 3 + flat.size
        words = total + (n32 + 1) // 2
        h64, h32 = self._upload.stage(words)
        h64[:total] = tokens
        o = 2 * total
        cu_q = h32[o:o + n + 1]
        cu_k = h32[o + n + 1:o + 2 * n + 2]
        cu_q[0] = cu_k[0] = 0
        np.cumsum(counts, out=cu_q[1:])
        np.cumsum(ends, out=cu_k[1:])
        h32[o + 2 * n + 2:o + 3 * n + 2] = starts
        h32[o + 3 * n + 2] = 0
        np.cumsum(t_counts, out=h32[o + 3 * n + 3:o + 4 * n + 3])
        h32[o + 4 * n + 3:o + n32] = flat
        # One fresh device buffer: the description, then ids and positions
        # (int64), then slots and the table (int32). Fresh per step, so the
        # tensors returned here stay valid after later steps.
        out_words = 2 * total + (total + n * width + 1) // 2
        buf = torch.empty(words + out_words, dtype=torch.int64, device=self.device)
        self._upload.commit(buf, words)
        d32 = buf.view(torch.int32)
        input_ids = buf[words:words + total]
        positions = buf[words + total:words + 2 * total]
        slots = d32[2 * (words + 2 * total):2 * (words + 2 * total) + total]
        t0 = 2 * (words + 2 * total) + total
        block_tables = d32[t0:t0 + n * width].view(n, width) if with_tables else None
        if n:
            self._launch(buf.data_ptr(), total, (0, 2 * n + 2, 3 * n + 2, 4 * n + 3), n, n,
                         total, None if block_tables is None else block_tables.data_ptr(),
                         width, width, None, slots.data_ptr(), positions.data_ptr(),
                         input_ids.data_ptr())
        metadata = AttentionMetadata.build(
            is_prefill=True,
            cu_seqlens_q=d32[o:o + n + 1],
            cu_seqlens_k=d32[o + n + 1:o + 2 * n + 2],
            max_seqlen_q=int(counts.max()) if n else 0,
            max_seqlen_k=int(ends.max()) if n else 0,
            slot_mapping=slots,
            block_tables=block_tables,
            validate_cache_write=self.debug_mode,
        )
        if self.debug_mode:
            self.validate(seqs, input_ids, positions, metadata, True)
        return input_ids, positions, metadata

    # -- decode ---------------------------------------------------------------
    def fill_decode(self, buffers: DecodeBuffers, seqs, rows: int | None = None) -> None:
        """Write one decode row per sequence (``_fill_decode_rows``,
        microinfer/runner.py:160-176) and, up to ``rows``, graph pad rows
        (``_fill_graph_bucket``, :561-576) into ``buffers``."""
        n = len(seqs)
        rows = n if rows is None else rows
        if rows < n or rows > buffers.capacity:
            raise ValueError("rows must cover the batch and fit the buffers")
        if rows > n and self.pad_block_id is None:
            raise ValueError("pad rows need a pad block")
        if rows and buffers.width < 1:
            raise ValueError("decode buffers need a table width of at least 1")
        tables = [s.block_table for s in seqs]
        counts = np.array([len(t) for t in tables], dtype=np.int64)
        flat = np.array(list(chain.from_iterable(tables)), dtype=np.int64)
        lengths = np.array([len(s) for s in seqs], dtype=np.int64)
        if n and (lengths < 1).any():
            raise ValueError("decode sequences must be nonempty")
        self._check_blocks(lengths - 1, counts, flat)
        needed = int(counts.max()) if n else 0
        if needed > buffers.width:
            raise ValueError("block table wider than the decode buffers")
        if rows > n:
            needed = max(needed, 1)

        # int32 words after the tokens: cu_q | starts | block offsets | blocks.
        n32 = 3 * n + 2 + flat.size
        words = n + (n32 + 1) // 2
        h64, h32 = self._upload.stage(words)
        h64[:n] = [s.last_token for s in seqs]
        o = 2 * n
        h32[o:o + n + 1] = np.arange(n + 1)
        h32[o + n + 1:o + 2 * n + 1] = lengths - 1
        h32[o + 2 * n + 1] = 0
        np.cumsum(counts, out=h32[o + 2 * n + 2:o + 3 * n + 2])
        h32[o + 3 * n + 2:o + n32] = flat
        dev = self._decode_upload
        if dev is None or dev.numel() < words:
            dev = torch.empty(max(words, 4096), dtype=torch.int64, device=self.device)
            self._decode_upload = dev
        self._upload.commit(dev, words)
        # Columns at or past buffers.table_written are -1 in every row, so only
        # the columns a row may still hold ids in are rewritten.
        cols = max(needed, buffers.table_written)
        self._launch(dev.data_ptr(), n, (0, n + 1, 2 * n + 1, 3 * n + 2), n, rows, rows,
                     buffers.block_tables.data_ptr(), buffers.width, cols,
                     buffers.context_lens.data_ptr(), buffers.slot_mapping.data_ptr(),
                     buffers.positions.data_ptr(), buffers.input_ids.data_ptr())
        buffers.table_written = needed if rows == buffers.capacity else cols

    def prepare_decode(self, seqs):
        """``ModelRunner.prepare_decode`` (microinfer/runner.py:348-385) on the device.

        The returned tensors are views of buffers reused by the next call,
        as in the reference.
        """
        n = len(seqs)
        width = max((len(s.block_table) for s in seqs), default=0)
        if self._decode_buffers is None:
            self._decode_buffers = DecodeBuffers(self.device)
        buffers = self._decode_buffers
        buffers.ensure(n, width)
        if n:
            self.fill_decode(buffers, seqs)
        metadata = AttentionMetadata.build(
            is_prefill=False,
            slot_mapping=buffers.slot_mapping[:n],
            context_lens=buffers.context_lens[:n],
            block_tables=buffers.block_tables[:n],
            validate_cache_write=self.debug_mode,
        )
        if self.debug_mode:
            self.validate(seqs, buffers.input_ids[:n], buffers.positions[:n], metadata, False)
        return buffers.input_ids[:n], buffers.positions[:n], metadata

    def validate(self, seqs, input_ids, positions, metadata, is_prefill: bool) -> None:
        """``validate_step`` with this builder's block size and limits."""
        validate_step(seqs, input_ids, positions, metadata, is_prefill, **self.limits)

    def pad_buffers(self, batch: int, width: int) -> DecodeBuffers:
        """Fresh bucket buffers holding only pad rows (``_fill_pad_buffers``,
        microinfer/runner.py:203-215)."""
        buffers = DecodeBuffers(self.device, batch, width)
        self.fill_decode(buffers, [], rows=batch)
        return buffers


class DecodeGraphRunner:
    """Graph-captured decode steps, one graph per batch bucket.

    Mirrors ``capture_cuda_graphs`` / ``_capture_bucket`` / ``_run_decode``
    (microinfer/runner.py:217-288, :555-604): each bucket has fixed buffers
    (table width ``num_blocks + 1``, so any sequence fits), filled with pad
    rows, warmed twice on a side stream and captured into one graph; all
    buckets share a memory pool. ``run`` picks the smallest bucket that holds
    the batch, writes the batch's rows and the pad rows on the device, replays
    and returns the first ``len(seqs)`` rows of the output.

    ``forward(input_ids, positions, metadata)`` is the step to capture (the
    model's decode forward, or here the attention layers); it must be
    capture-safe. With ``greedy`` its output is ``[batch, vocab]`` logits and
    the graph also selects each row's greedy token with the HIP argmax
    (runner.py:236-240); ``run`` then returns ``(logits, tokens)`` like
    ``_run_decode`` (runner.py:603).
    """

    def __init__(self, builder: StepMetadataBuilder, forward, *, max_num_seqs: int,
                 table_width: int, greedy: bool = False):
        if builder.pad_block_id is None:
            raise ValueError("graph buckets need the builder's pad block")
        if builder.device.type != "cuda":
            raise RuntimeError("graph capture needs a HIP device")
        self.builder = builder
        self.forward = forward
        self.greedy = greedy
        self.table_width = table_width
        self.buckets = []
        self.pool = None
        for batch in graph_buckets(max_num_seqs):
            self._capture(batch)

    def _capture(self, batch: int) -> None:
        device = self.builder.device
        buffers = self.builder.pad_buffers(batch, self.table_width)
        ids, positions = buffers.input_ids[:batch], buffers.positions[:batch]
        torch.cuda.synchronize(device)
        side = torch.cuda.Stream(device=device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side), torch.inference_mode():
            for _ in range(2):
                self._step(ids, positions, buffers.metadata(batch))
        torch.cuda.current_stream(device).wait_stream(side)
        torch.cuda.synchronize(device)
        graph = torch.cuda.CUDAGraph()
        # Captured on the warm-up stream, so per-stream state the library
        # created during the warm-up (the decode arrival counters, the argmax
        # row slots) is reused rather than allocated and zero-filled inside
        # the graph.
        with capture_graph(graph, self.pool, stream=side), torch.inference_mode():
            out = self._step(ids, positions, buffers.metadata(batch))
        if self.pool is None:
            self.pool = graph.pool()
        torch.cuda.synchronize(device)
        self.buckets.append((batch, buffers, graph, out))

    def _step(self, ids, positions, metadata):
        out = self.forward(ids, positions, metadata)
        return (out, greedy_argmax(out)) if self.greedy else out

    def select(self, batch: int):
        for bucket in self.buckets:
            if bucket[0] >= batch:
                return bucket
        return None

    def run(self, seqs):
        """Replay the bucket that holds ``seqs``; None if the batch is larger
        than every bucket (the caller then runs eagerly, as the reference does)."""
        bucket = self.select(len(seqs))
        if bucket is None:
            return None
        batch, buffers, graph, out = bucket
        self.builder.fill_decode(buffers, seqs, rows=batch)
        n = len(seqs)
        if self.builder.debug_mode:
            # The batch's rows as the graph will read them (microinfer/
            # runner.py:582-598).
            self.builder.validate(seqs, buffers.input_ids[:n], buffers.positions[:n],
                                  buffers.metadata(n), False)
        graph.replay()
        if self.greedy:
            return out[0][:n], out[1][:n]
        return out[:n]

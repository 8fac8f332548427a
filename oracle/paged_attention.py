"""numpy restatement of MicroInfer's CPU paged-attention path (test infrastructure).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this module. It is what results are compared with, never the thing measured or
shipped.

Layout conventions follow the reference exactly:

* ``query``       ``[T, Hq, D]`` float (already widened to float32/float64)
* ``key_cache``   ``[N, B, Hkv, D]`` (physical blocks x tokens-in-block)
* ``block_tables````[R, W]`` integer, ``-1`` padded
* ``context_lens`` per-request context length ``c`` (includes the new tokens)
* ``cu_seqlens_q````[R + 1]`` prefix sums of query lengths

How each function is pinned (tests/test_oracle_*.py):

* ``paged_attention_reference`` -- the reference's own known answers
  (tests/components/test_paged_attention.py:49-64 -> [[3,3]],[[10,10]];
  :82-103 -> uniform 3.0 without half overflow), its in-test dense loop
  (:10-46, physical order [2,0], +-1000 poison), a float64 textbook brute force
  written with explicit loops (``dense_causal_attention_f64``), invariants
  (chunked + decode == full prefill as in test_cache_binding.py:102-133, packed
  == separate, permutation of physical blocks, poison never read) and closed
  forms (constant V rows -> output equals that constant; one visible key ->
  output equals its V row).
* ``kv_append`` / ``slot_indices`` / ``gather_paged_kv`` -- the reference's
  known answers (test_kv_cache.py:10-33: arange 0..29 into slots
  [8,9,10,11,0] read back through table [2,0]; slot -1 skipped;
  test_metadata.py:40-57: slots [0,5,2] -> blocks [0,1,0], offsets [0,1,2]
  at B=4 and [0,2,1]/[0,1,0] at B=2) and byte-exact brute force.
* ``merge_partials`` / ``partial_attention_states`` -- merging any partition of
  the context must reproduce the single-pass result; an empty partition
  (m=-inf, l=0) contributes nothing.
"""

from __future__ import annotations

import math

import numpy as np


def slot_indices(slot_mapping, block_size: int):
    """(block, offset) of each slot, floor semantics.

    Follows ``AttentionMetadata.slot_indices`` (microinfer/layer/metadata.py:75-84):
    ``blocks = floor(slot / B)``, ``offsets = slot - blocks * B``.
    """
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    slots = np.asarray(slot_mapping, dtype=np.int64)
    blocks = np.floor_divide(slots, block_size)
    return blocks, slots - blocks * block_size


def kv_append(key_cache, value_cache, slot_mapping, keys, values, *, skip_negative=True):
    """Scatter new K/V rows into the paged cache in place.

    Follows ``LayerKVCache.write_checked``/``write_fast``
    (microinfer/worker/kv_cache.py:30-79): slot ``s`` writes
    ``cache[s // B, s % B] = row``; slots equal to -1 are padding and are
    skipped (write_checked, :42). Works on any numpy dtype, bit for bit
    (bf16 caches travel as uint16).
    """
    block_size = key_cache.shape[1]
    slots = np.asarray(slot_mapping, dtype=np.int64)
    valid = slots >= 0 if skip_negative else np.ones(slots.shape, dtype=bool)
    blocks, offsets = slot_indices(slots[valid], block_size)
    key_cache[blocks, offsets] = np.asarray(keys)[valid]
    value_cache[blocks, offsets] = np.asarray(values)[valid]


def gather_paged_kv(key_cache, value_cache, block_tables, contexts, block_size):
    """Concatenate each request's valid cache rows into varlen K/V.

    Follows ``_gather_paged_kv`` (microinfer/layer/paged_attention.py:76-101):
    for request r take ``ceil(c_r / B)`` table entries, index the cache, flatten
    to ``[-1, Hkv, D]`` and keep the first ``c_r`` rows; concatenate requests.
    """
    num_kv_heads, head_dim = key_cache.shape[2], key_cache.shape[3]
    keys, values = [], []
    for request, context_len in enumerate(contexts):
        num_blocks = (context_len + block_size - 1) // block_size
        blocks = np.asarray(block_tables[request][:num_blocks], dtype=np.int64)
        keys.append(key_cache[blocks].reshape(-1, num_kv_heads, head_dim)[:context_len])
        values.append(
            value_cache[blocks].reshape(-1, num_kv_heads, head_dim)[:context_len]
        )
    if not keys:
        empty = np.empty((0, num_kv_heads, head_dim), dtype=key_cache.dtype)
        return empty, empty.copy()
    return np.concatenate(keys), np.concatenate(values)


def paged_attention_reference(
    query,
    key_cache,
    value_cache,
    block_tables,
    context_lens,
    cu_seqlens_q,
    *,
    scale: float,
    accumulation=np.float32,
):
    """Causal GQA attention over a paged cache, one request at a time.

    Follows ``_paged_attention_reference`` (microinfer/layer/paged_attention.py:22-67):

    * gather ``K, V = cache[table[r, :ceil(c/B)]]`` -> ``[c, Hkv, D]`` (:43-46);
    * queries ``[q, Hkv, G, D]`` with ``G = Hq / Hkv`` so query head ``h`` reads
      KV head ``h // G`` (:51-55);
    * ``S = (Q K^T) * scale`` in the accumulation dtype (:56, :62);
    * bottom-right causal mask: query i sits at position ``(c - q_len) + i`` and
      sees keys ``k_pos <= q_pos`` (:57-62);
    * softmax over keys, then ``P V`` (:63).

    Inputs are float arrays (bf16/fp16 data already widened); the result is in
    ``accumulation`` dtype -- the caller rounds to the activation dtype, as the
    reference does with ``.to(query.dtype)`` (:65). Requests with no context
    produce zeros (the reference's ``torch.zeros_like`` result, :35).
    """
    query = np.asarray(query, dtype=accumulation)
    key_cache = np.asarray(key_cache)
    value_cache = np.asarray(value_cache)
    _total, num_q_heads, head_dim = query.shape
    _blocks, block_size, num_kv_heads, _ = key_cache.shape
    group = num_q_heads // num_kv_heads
    result = np.zeros_like(query)
    for request in range(len(context_lens)):
        context_len = int(context_lens[request])
        start, end = int(cu_seqlens_q[request]), int(cu_seqlens_q[request + 1])
        if end == start or context_len <= 0:
            continue
        num_blocks = (context_len + block_size - 1) // block_size
        blocks = np.asarray(block_tables[request][:num_blocks], dtype=np.int64)
        keys = key_cache[blocks].reshape(-1, num_kv_heads, head_dim)[:context_len]
        values = value_cache[blocks].reshape(-1, num_kv_heads, head_dim)[:context_len]
        keys = keys.astype(accumulation)  # [c, Hkv, D]
        values = values.astype(accumulation)
        q = query[start:end].reshape(-1, num_kv_heads, group, head_dim)
        # einsum("qhgd,khd->hgqk") as a batched matmul over KV heads.
        q_hg = q.transpose(1, 2, 0, 3)  # [Hkv, G, q, D]
        k_hd = keys.transpose(1, 2, 0)[:, None]  # [Hkv, 1, D, c]
        scores = np.matmul(q_hg, k_hd) * accumulation(scale)  # [Hkv, G, q, c]
        prefix = context_len - (end - start)
        q_pos = prefix + np.arange(end - start)
        k_pos = np.arange(context_len)
        visible = q_pos[:, None] >= k_pos[None, :]
        scores = np.where(visible, scores, -np.inf)
        row_max = scores.max(axis=-1, keepdims=True)
        row_max = np.where(np.isfinite(row_max), row_max, 0)
        weights = np.exp(scores - row_max)
        weights /= weights.sum(axis=-1, keepdims=True)
        v_hd = values.transpose(1, 0, 2)[:, None]  # [Hkv, 1, c, D]
        out = np.matmul(weights, v_hd)  # [Hkv, G, q, D]
        result[start:end] = out.transpose(2, 0, 1, 3).reshape(-1, num_q_heads, head_dim)
    return result


def dense_causal_attention_f64(query, keys, values, *, scale: float, prefix: int = 0):
    """Textbook causal GQA attention with explicit loops, in float64.

    ``query [q, Hq, D]`` over logical ``keys/values [c, Hkv, D]`` with
    ``c = prefix + q``. Independent of any paging: used to pin
    ``paged_attention_reference`` (mirrors the dense loop of
    tests/components/test_paged_attention.py:26-33). Small inputs only.
    """
    query = np.asarray(query, dtype=np.float64)
    keys = np.asarray(keys, dtype=np.float64)
    values = np.asarray(values, dtype=np.float64)
    q_len, num_q_heads, head_dim = query.shape
    num_kv_heads = keys.shape[1]
    group = num_q_heads // num_kv_heads
    out = np.zeros((q_len, num_q_heads, head_dim), dtype=np.float64)
    for i in range(q_len):
        visible = prefix + i + 1
        for head in range(num_q_heads):
            kv = head // group
            logits = [
                sum(query[i, head, d] * keys[j, kv, d] for d in range(head_dim)) * scale
                for j in range(visible)
            ]
            top = max(logits)
            exps = [math.exp(x - top) for x in logits]
            total = sum(exps)
            for d in range(head_dim):
                out[i, head, d] = sum(exps[j] * values[j, kv, d] for j in range(visible)) / total
    return out


def partial_attention_states(query_row, keys, values, *, scale: float, bounds):
    """Unnormalised online-softmax state of one query row over key ranges.

    For each ``[lo, hi)`` in ``bounds`` return ``(acc, m, l)`` with natural-log
    max ``m = max_j s_j``, ``l = sum_j exp(s_j - m)`` and
    ``acc = sum_j exp(s_j - m) v_j`` -- the per-split state the reference's
    decode kernel emits (microinfer/layer/triton_paged_attention.py:116-131).
    ``query_row [Hq, D]``, ``keys/values [c, Hkv, D]``. Empty ranges give
    ``(0, -inf, 0)``.
    """
    query_row = np.asarray(query_row, dtype=np.float64)
    keys = np.asarray(keys, dtype=np.float64)
    values = np.asarray(values, dtype=np.float64)
    num_q_heads, head_dim = query_row.shape
    group = num_q_heads // keys.shape[1]
    states = []
    for lo, hi in bounds:
        acc = np.zeros((num_q_heads, head_dim))
        m = np.full(num_q_heads, -np.inf)
        l = np.zeros(num_q_heads)
        for head in range(num_q_heads):
            if hi <= lo:
                continue
            k = keys[lo:hi, head // group]
            v = values[lo:hi, head // group]
            s = (k @ query_row[head]) * scale
            m[head] = s.max()
            p = np.exp(s - m[head])
            l[head] = p.sum()
            acc[head] = p @ v
        states.append((acc, m, l))
    return states


def merge_partials(states):
    """Combine split states: ``out = sum w_i acc_i / sum w_i l_i``, ``w_i = e^(m_i - g)``.

    Follows ``_paged_decode_reduce_kernel``
    (microinfer/layer/triton_paged_attention.py:244-257); empty splits
    (m = -inf, l = 0) get weight zero.
    """
    acc = np.stack([s[0] for s in states])  # [S, Hq, D]
    m = np.stack([s[1] for s in states])  # [S, Hq]
    l = np.stack([s[2] for s in states])
    g = m.max(axis=0)
    safe_g = np.where(np.isfinite(g), g, 0.0)
    w = np.where(np.isfinite(m), np.exp(m - safe_g), 0.0)
    numerator = (acc * w[..., None]).sum(axis=0)
    denominator = (l * w).sum(axis=0)
    return numerator / denominator[..., None]

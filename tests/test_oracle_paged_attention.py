"""Pin the attention oracle against the reference's own tests and mathematics.

Restates tests/components/test_paged_attention.py:10-103 and the chunked/packed
invariants of test_cache_binding.py:102-133 and test_model_cache.py:45-77
against ``oracle.paged_attention_reference``, plus a float64 textbook brute
force, closed forms and planted mistakes that these checks must catch.
"""

import math

import numpy as np
import pytest

from oracle import (
    dense_causal_attention_f64,
    merge_partials,
    paged_attention_reference,
    partial_attention_states,
    round_to_dtype,
)

DTYPES = ["f32", "f16", "bf16"]


def scatter_paged(logical_k, logical_v, table, num_blocks, block_size, poison=1000.0):
    heads, dim = logical_k.shape[1:]
    k = np.full((num_blocks, block_size, heads, dim), poison, dtype=np.float32)
    v = np.full_like(k, -poison)
    for pos in range(len(logical_k)):
        k[table[pos // block_size], pos % block_size] = logical_k[pos]
        v[table[pos // block_size], pos % block_size] = logical_v[pos]
    return k, v


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("prefix,query_len", [(0, 3), (2, 1), (1, 2)])
def test_paged_causal_gqa_matches_dense_loop(prefix, query_len, dtype):
    # test_paged_attention.py:10-46: physical order [2, 0], poison +-1000.
    rng = np.random.default_rng(0)
    context = prefix + query_len
    q = round_to_dtype(rng.standard_normal((query_len, 4, 4)), dtype)
    logical_k = round_to_dtype(rng.standard_normal((context, 2, 4)), dtype)
    logical_v = round_to_dtype(rng.standard_normal((context, 2, 4)), dtype)
    table = [2, 0]
    k, v = scatter_paged(logical_k, logical_v, table, 3, 2)
    expected = np.empty((query_len, 4, 4), dtype=np.float32)
    for qi in range(query_len):
        visible = prefix + qi + 1
        for head in range(4):
            kh = logical_k[:visible, head // 2]
            vh = logical_v[:visible, head // 2]
            logits = kh @ q[qi, head] / 2
            p = np.exp(logits - logits.max())
            expected[qi, head] = (p / p.sum()) @ vh
    actual = paged_attention_reference(q, k, v, [table], [context], [0, query_len], scale=0.5)
    actual = round_to_dtype(actual, dtype)
    tolerance = 1e-5 if dtype == "f32" else 1e-2
    np.testing.assert_allclose(actual, expected, atol=tolerance, rtol=tolerance)


def test_requests_cannot_attend_to_each_other_or_padding():
    # test_paged_attention.py:49-64 known answer.
    q = np.zeros((2, 1, 2), np.float32)
    k = np.zeros((3, 2, 1, 2), np.float32)
    v = np.full_like(k, 999)
    v[2, 0] = 2
    v[2, 1] = 4
    v[0, 0] = 10
    out = paged_attention_reference(
        q, k, v, [[2, -1], [0, -1]], [2, 1], [0, 1, 2], scale=1 / math.sqrt(2)
    )
    np.testing.assert_array_equal(out, np.array([[[3.0, 3.0]], [[10.0, 10.0]]], np.float32))


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_large_scores_do_not_overflow(dtype):
    # test_paged_attention.py:82-103: logits 1000*1000*4 -> uniform 3.0.
    q = round_to_dtype(np.full((1, 2, 4), 1000.0), dtype)
    k = round_to_dtype(np.full((1, 2, 1, 4), 1000.0), dtype)
    v = np.broadcast_to(np.array([2.0, 4.0], np.float32).reshape(1, 2, 1, 1), k.shape)
    out = paged_attention_reference(q, k, v, [[0]], [2], [0, 1], scale=0.5)
    np.testing.assert_allclose(round_to_dtype(out, dtype), np.full((1, 2, 4), 3.0))


@pytest.mark.parametrize("seed", range(4))
def test_matches_float64_brute_force(seed):
    rng = np.random.default_rng(seed)
    heads_q, heads_kv, dim, block = [(4, 2, 8, 4), (6, 3, 4, 2), (8, 1, 16, 8), (3, 3, 4, 4)][seed]
    prefix, q_len = int(rng.integers(0, 9)), int(rng.integers(1, 6))
    context = prefix + q_len
    q = rng.standard_normal((q_len, heads_q, dim)).astype(np.float32)
    lk = rng.standard_normal((context, heads_kv, dim)).astype(np.float32)
    lv = rng.standard_normal((context, heads_kv, dim)).astype(np.float32)
    blocks = (context + block - 1) // block
    table = list(rng.permutation(blocks + 3)[:blocks])
    k, v = scatter_paged(lk, lv, table, blocks + 3, block)
    scale = 1 / math.sqrt(dim)
    expected = dense_causal_attention_f64(q, lk, lv, scale=scale, prefix=prefix)
    actual = paged_attention_reference(q, k, v, [table], [context], [0, q_len], scale=scale)
    np.testing.assert_allclose(actual, expected, atol=1e-5, rtol=1e-5)


def test_chunked_prefill_plus_decode_equals_full():
    # test_cache_binding.py:102-133: chunks (0-3), (3-5) and decode (5-6) over
    # physical blocks 2, 0, 3 equal one full causal pass.
    rng = np.random.default_rng(1)
    q = rng.standard_normal((6, 4, 4)).astype(np.float32)
    lk = rng.standard_normal((6, 2, 4)).astype(np.float32)
    lv = rng.standard_normal((6, 2, 4)).astype(np.float32)
    k, v = scatter_paged(lk, lv, [2, 0, 3], 4, 2)
    full = paged_attention_reference(q, k, v, [[2, 0, 3]], [6], [0, 6], scale=0.5)
    pieces = [
        paged_attention_reference(q[a:b], k, v, [[2, 0, 3]], [b], [0, b - a], scale=0.5)
        for a, b in [(0, 3), (3, 5), (5, 6)]
    ]
    np.testing.assert_allclose(np.concatenate(pieces), full, atol=1e-6)
    dense = dense_causal_attention_f64(q, lk, lv, scale=0.5)
    np.testing.assert_allclose(full, dense, atol=1e-5)


def test_packed_requests_equal_separate_and_ignore_poison():
    rng = np.random.default_rng(2)
    lk_a, lv_a = rng.standard_normal((2, 5, 2, 8)).astype(np.float32)
    lk_b, lv_b = rng.standard_normal((2, 3, 2, 8)).astype(np.float32)
    k = np.full((6, 4, 2, 8), np.nan, np.float32)
    v = np.full_like(k, np.nan)
    for pos in range(5):
        k[[4, 1][pos // 4], pos % 4], v[[4, 1][pos // 4], pos % 4] = lk_a[pos], lv_a[pos]
    for pos in range(3):
        k[5, pos], v[5, pos] = lk_b[pos], lv_b[pos]
    q = rng.standard_normal((3, 4, 8)).astype(np.float32)  # 2 rows for a, 1 for b
    tables = [[4, 1], [5, -1]]
    packed = paged_attention_reference(q, k, v, tables, [5, 3], [0, 2, 3], scale=0.3)
    a = paged_attention_reference(q[:2], k, v, tables[:1], [5], [0, 2], scale=0.3)
    b = paged_attention_reference(q[2:], k, v, tables[1:], [3], [0, 1], scale=0.3)
    assert np.isfinite(packed).all()
    np.testing.assert_array_equal(packed, np.concatenate([a, b]))


def test_physical_block_permutation_invariance():
    rng = np.random.default_rng(3)
    lk = rng.standard_normal((11, 2, 4)).astype(np.float32)
    lv = rng.standard_normal((11, 2, 4)).astype(np.float32)
    q = rng.standard_normal((1, 4, 4)).astype(np.float32)
    outs = []
    for table in ([0, 1, 2], [2, 0, 1], [5, 3, 4]):
        k, v = scatter_paged(lk, lv, table, 6, 4)
        outs.append(paged_attention_reference(q, k, v, [table], [11], [0, 1], scale=0.5))
    np.testing.assert_allclose(outs[1], outs[0], atol=1e-6)
    np.testing.assert_allclose(outs[2], outs[0], atol=1e-6)


def test_closed_forms():
    rng = np.random.default_rng(4)
    q = rng.standard_normal((1, 4, 8)).astype(np.float32)
    # Constant V rows: every softmax-weighted average equals that constant.
    k = rng.standard_normal((2, 4, 2, 8)).astype(np.float32)
    v = np.broadcast_to(np.arange(8, dtype=np.float32), (2, 4, 2, 8)).copy()
    out = paged_attention_reference(q, k, v, [[1, 0]], [7], [0, 1], scale=0.3)
    np.testing.assert_allclose(out, np.broadcast_to(np.arange(8.0), (1, 4, 8)), atol=1e-5)
    # One visible key: output equals that key's V row (per KV head).
    v = rng.standard_normal((2, 4, 2, 8)).astype(np.float32)
    out = paged_attention_reference(q, k, v, [[1]], [1], [0, 1], scale=0.3)
    expected = np.stack([v[1, 0, h // 2] for h in range(4)])[None]
    np.testing.assert_allclose(out, expected, atol=1e-6)
    # Zero context produces zeros.
    out = paged_attention_reference(q, k, v, [[1]], [0], [0, 1], scale=0.3)
    assert (out == 0).all()


@pytest.mark.parametrize("bounds", [[(0, 13)], [(0, 5), (5, 13)], [(0, 0), (0, 7), (7, 7), (7, 13)],
                                    [(i, i + 1) for i in range(13)]])
def test_split_merge_equals_single_pass(bounds):
    rng = np.random.default_rng(5)
    q = rng.standard_normal((4, 8))
    keys = rng.standard_normal((13, 2, 8))
    values = rng.standard_normal((13, 2, 8))
    merged = merge_partials(partial_attention_states(q, keys, values, scale=0.4, bounds=bounds))
    single = dense_causal_attention_f64(q[None], keys, values, scale=0.4, prefix=12)[0]
    np.testing.assert_allclose(merged, single, atol=1e-12)


def _plant(name):
    """Plausible oracle mistakes; each must fail the checks above."""
    def wrong_head_map(q, k, v, tables, contexts, cu_q, *, scale):
        # Interleaved GQA mapping (h % Hkv instead of h // G).
        reordered = q.reshape(q.shape[0], -1, k.shape[2], q.shape[2]).transpose(0, 2, 1, 3)
        reordered = reordered.reshape(q.shape)
        return paged_attention_reference(reordered, k, v, tables, contexts, cu_q, scale=scale)

    def top_left_mask(q, k, v, tables, contexts, cu_q, *, scale):
        # Causal mask aligned to the first key instead of the last.
        out = np.zeros_like(q)
        for r in range(len(contexts)):
            a, b = cu_q[r], cu_q[r + 1]
            out[a:b] = paged_attention_reference(
                q[a:b], k, v, [tables[r]], [b - a], [0, b - a], scale=scale
            )
        return out

    return {"head_map": wrong_head_map, "mask": top_left_mask}[name]


@pytest.mark.parametrize("mistake", ["head_map", "mask"])
def test_planted_mistakes_are_caught(mistake):
    rng = np.random.default_rng(6)
    prefix, q_len = 3, 2
    q = rng.standard_normal((q_len, 4, 4)).astype(np.float32)
    lk = rng.standard_normal((prefix + q_len, 2, 4)).astype(np.float32)
    lv = rng.standard_normal((prefix + q_len, 2, 4)).astype(np.float32)
    k, v = scatter_paged(lk, lv, [2, 0, 1], 3, 2)
    expected = dense_causal_attention_f64(q, lk, lv, scale=0.5, prefix=prefix)
    wrong = _plant(mistake)(q, k, v, [[2, 0, 1]], [prefix + q_len], [0, q_len], scale=0.5)
    assert np.abs(wrong - expected).max() > 1e-2

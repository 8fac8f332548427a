"""Paged decode on the GPU against the oracle.

Restates tests/layers/test_triton_paged_attention.py:14-77 and the decode
half of tests/components/test_paged_attention.py, then runs the decode
workloads at their real sizes (0.6B and 8B attention shapes) and the
properties the path must keep: split-plan invariance, GQA group sizes,
head dims, empty and one-token contexts, poison never read, masked invalid
table entries, and hipGraph replay with changing contexts.

Tolerances (max-abs against the fp32 oracle): 1e-5 on the reference's own
small fp32 cases, 2e-3 fp32 / 2e-2 bf16 and fp16 elsewhere.
"""

import math

import numpy as np
import pytest
import torch

from microinfer_amd.layer.hip_paged_attention import hip_paged_decode
from microinfer_amd.runner import capture_graph
from microinfer_amd.worker.kv_cache import KVCache
from microinfer_amd.workloads import QWEN3_06B, QWEN3_8B, make_decode_batch
from oracle import kv_append
from tests.support import (
    TOLERANCE,
    as_f32,
    bits,
    checked_paged_attention,
    max_abs,
    oracle_attention,
    oracle_decode,
    rounded,
)

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("block_size", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_decode_matches_reference_small(block_size, dtype):
    # test_triton_paged_attention.py:14-77: reversed physical blocks.
    torch.manual_seed(0)
    requests, hq, hkv, d = 2, 4, 2, 32
    contexts = [5, block_size + 3]
    nb = (max(contexts) + block_size - 1) // block_size
    physical = list(range(requests * nb))[::-1]
    tables = torch.tensor([physical[:nb], physical[nb : 2 * nb]], dtype=torch.int32, device=DEV)
    kc = torch.randn(requests * nb, block_size, hkv, d, device=DEV, dtype=dtype)
    vc = torch.randn_like(kc)
    q = torch.randn(requests, hq, d, device=DEV, dtype=dtype)
    scale = 1 / d**0.5
    expected = oracle_attention(q, kc, vc, tables, contexts, [0, 1, 2], scale)
    actual = hip_paged_decode(q, kc, vc, tables, torch.tensor(contexts, dtype=torch.int32, device=DEV),
                              scale=scale)
    assert actual.dtype == dtype
    tolerance = 1e-5 if dtype == torch.float32 else 2e-2
    np.testing.assert_allclose(as_f32(actual), expected, atol=tolerance, rtol=tolerance)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("layout", ["paired", "head_major", "token_major"])
def test_small_decode_workload_append_then_attend(dtype, layout):
    # 0.6B layer, pool 1024, 8 sequences, contexts U[64, 512], seed 0: the
    # append writes position c-1, then attention reads all c tokens.
    batch = make_decode_batch(num_seqs=8, ctx_lo=64, ctx_hi=512, pool_blocks=1024, **QWEN3_06B)
    cache = KVCache(1, 1024, 16, 8, 128, dtype=dtype, device=DEV, layout=layout)
    cache.keys[0].copy_(rounded(batch.key_pool, dtype, DEV))
    cache.values[0].copy_(rounded(batch.value_pool, dtype, DEV))
    view = cache.layer(0)
    new_k = rounded(batch.new_keys, dtype, DEV)
    new_v = rounded(batch.new_values, dtype, DEV)
    expected_k, expected_v = bits(view.keys), bits(view.values)
    view.write_slots(torch.tensor(batch.slots, dtype=torch.int32, device=DEV), new_k, new_v)
    kv_append(expected_k, expected_v, batch.slots, bits(new_k), bits(new_v))
    assert np.array_equal(bits(view.keys), expected_k)
    q = rounded(batch.query, dtype, DEV)
    tables = torch.tensor(batch.block_tables, device=DEV)
    lens = torch.tensor(batch.context_lens, device=DEV)
    scale = 1 / math.sqrt(128)
    out = hip_paged_decode(q, view.keys, view.values, tables, lens, scale=scale)
    expected = oracle_decode(q, view.keys, view.values, tables, lens, scale)
    assert max_abs(out, expected) <= TOLERANCE[dtype]


@pytest.mark.parametrize("layout", ["paired", "head_major", "token_major"])
def test_decode_batch32_workload(layout):
    # 0.6B shape, bf16, pool 16384, 32 sequences, contexts U[128, 2048].
    batch = make_decode_batch(num_seqs=32, ctx_lo=128, ctx_hi=2048, pool_blocks=16384,
                              draw_pools=False, **QWEN3_06B)
    cache = KVCache(1, 16384, 16, 8, 128, dtype=torch.bfloat16, device=DEV, layout=layout)
    gen = torch.Generator(device=DEV).manual_seed(0)
    cache.keys[0].copy_(torch.randn(cache.keys[0].shape, generator=gen, device=DEV))
    cache.values[0].copy_(torch.randn(cache.values[0].shape, generator=gen, device=DEV))
    q = rounded(batch.query, torch.bfloat16, DEV)
    tables = torch.tensor(batch.block_tables, device=DEV)
    lens = torch.tensor(batch.context_lens, device=DEV)
    scale = 1 / math.sqrt(128)
    out = hip_paged_decode(q, cache.keys[0], cache.values[0], tables, lens, scale=scale)
    expected = oracle_decode(q, cache.keys[0], cache.values[0], tables, lens, scale)
    assert max_abs(out, expected) <= 2e-2


@pytest.mark.parametrize(
    "num_seqs,context",
    [(1, 4096), (1, 16384), (1, 32768), (4, 4096), (4, 16384), (4, 32768)],
)
def test_long_context_split_decode(num_seqs, context):
    # 8B shape (32 Q / 8 KV heads), bf16, pool 65536 blocks, fixed contexts:
    # every point of the long-context grid (1 or 4 sequences x 4K / 16K / 32K).
    batch = make_decode_batch(num_seqs=num_seqs, ctx_lo=context, ctx_hi=context,
                              pool_blocks=65536, draw_pools=False, **QWEN3_8B)
    cache = KVCache(1, 65536, 16, 8, 128, dtype=torch.bfloat16, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(0)
    cache.keys[0].copy_(torch.randn(cache.keys[0].shape, generator=gen, device=DEV))
    cache.values[0].copy_(torch.randn(cache.values[0].shape, generator=gen, device=DEV))
    q = rounded(batch.query, torch.bfloat16, DEV)
    tables = torch.tensor(batch.block_tables, device=DEV)
    lens = torch.tensor(batch.context_lens, device=DEV)
    scale = 1 / math.sqrt(128)
    out = hip_paged_decode(q, cache.keys[0], cache.values[0], tables, lens, scale=scale)
    expected = oracle_decode(q, cache.keys[0], cache.values[0], tables, lens, scale)
    assert max_abs(out, expected) <= 2e-2


@pytest.mark.parametrize("split_k", [1, 2, 4, 16, 64])
def test_split_plan_invariance(split_k):
    rng = np.random.default_rng(3)
    contexts = [1, 15, 16, 17, 300, 1000]
    tables = torch.tensor(
        np.stack([rng.permutation(256)[:64] for _ in contexts]).astype(np.int32), device=DEV
    )
    kc = torch.randn(256, 16, 2, 64, device=DEV)
    vc = torch.randn_like(kc)
    q = torch.randn(6, 8, 64, device=DEV)
    lens = torch.tensor(contexts, dtype=torch.int32, device=DEV)
    adaptive = hip_paged_decode(q, kc, vc, tables, lens)
    forced = hip_paged_decode(q, kc, vc, tables, lens, split_k=split_k)
    expected = oracle_decode(q, kc, vc, tables, lens, 1 / 8)
    assert max_abs(adaptive, expected) <= 1e-5
    assert max_abs(forced, expected) <= 1e-5


@pytest.mark.parametrize("hq,hkv", [(8, 8), (8, 4), (12, 4), (16, 4), (20, 4), (24, 4), (32, 4),
                                    (28, 4), (32, 8)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gqa_group_sizes(hq, hkv, dtype):
    torch.manual_seed(1)
    d, bs = 128, 16
    contexts = [37, 300, 129]
    tables = torch.arange(3 * 19, dtype=torch.int32, device=DEV).reshape(3, 19).flip(-1).contiguous()
    kc = torch.randn(57, bs, hkv, d, device=DEV).to(dtype)
    vc = torch.randn_like(kc)
    q = torch.randn(3, hq, d, device=DEV).to(dtype)
    lens = torch.tensor(contexts, dtype=torch.int32, device=DEV)
    out = hip_paged_decode(q, kc, vc, tables, lens)
    expected = oracle_decode(q, kc, vc, tables, lens, 1 / math.sqrt(d))
    assert max_abs(out, expected) <= TOLERANCE[dtype]


@pytest.mark.parametrize("head_dim", [2, 4, 8, 16, 32, 64, 256])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_head_dims(head_dim, dtype):
    torch.manual_seed(2)
    contexts = [3, 40, 77]
    tables = torch.tensor([[4, 0, 2, 7, 9, 1], [3, 5, 6, 8, 10, 11], [12, 13, 14, 15, 16, 17]],
                          dtype=torch.int32, device=DEV)
    kc = torch.randn(18, 16, 2, head_dim, device=DEV).to(dtype)
    vc = torch.randn_like(kc)
    q = torch.randn(3, 4, head_dim, device=DEV).to(dtype)
    lens = torch.tensor(contexts, dtype=torch.int32, device=DEV)
    out = hip_paged_decode(q, kc, vc, tables, lens)
    expected = oracle_decode(q, kc, vc, tables, lens, 1 / math.sqrt(head_dim))
    assert max_abs(out, expected) <= TOLERANCE[dtype]


def test_known_answers_and_edge_contexts():
    # test_paged_attention.py:49-64: isolated requests, padding ignored.
    q = torch.zeros(2, 1, 2, device=DEV)
    k = torch.zeros(3, 2, 1, 2, device=DEV)
    v = torch.full_like(k, 999)
    v[2, 0] = 2
    v[2, 1] = 4
    v[0, 0] = 10
    out = checked_paged_attention(q, k, v, torch.tensor([[2, -1], [0, -1]], device=DEV),
                                  torch.tensor([2, 1], device=DEV), torch.tensor([0, 1, 2], device=DEV))
    assert torch.equal(out.cpu(), torch.tensor([[[3.0, 3.0]], [[10.0, 10.0]]]))
    # Zero context -> zeros; one token -> its V row.
    kc = torch.randn(4, 16, 2, 32, device=DEV)
    vc = torch.randn_like(kc)
    qq = torch.randn(2, 4, 32, device=DEV)
    tables = torch.tensor([[1, 2], [3, 0]], dtype=torch.int32, device=DEV)
    out = hip_paged_decode(qq, kc, vc, tables, torch.tensor([0, 1], dtype=torch.int32, device=DEV))
    assert (out[0] == 0).all()
    assert torch.allclose(out[1], vc[3, 0].repeat_interleave(2, dim=0), atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_large_logits_do_not_overflow(dtype):
    # test_paged_attention.py:82-103.
    query = torch.full((1, 2, 4), 1000.0, dtype=dtype, device=DEV)
    keys = torch.full((1, 2, 1, 4), 1000.0, dtype=dtype, device=DEV)
    values = torch.tensor([2.0, 4.0], dtype=dtype, device=DEV).reshape(1, 2, 1, 1).expand_as(keys)
    out = checked_paged_attention(query, keys, values.contiguous(), torch.tensor([[0]], device=DEV),
                                  torch.tensor([2], device=DEV), torch.tensor([0, 1], device=DEV))
    assert torch.equal(out.float().cpu(), torch.full((1, 2, 4), 3.0))


def test_poison_is_never_read_and_bad_table_entries_are_masked():
    torch.manual_seed(4)
    kc = torch.full((8, 16, 2, 64), float("nan"), device=DEV)
    vc = torch.full_like(kc, float("nan"))
    contexts = [20, 33]
    tables = torch.tensor([[5, 2, -1, -1], [0, 7, 3, -1]], dtype=torch.int32, device=DEV)
    for r, c in enumerate(contexts):
        for pos in range(c):
            blk = int(tables[r, pos // 16])
            kc[blk, pos % 16] = torch.randn(2, 64, device=DEV)
            vc[blk, pos % 16] = torch.randn(2, 64, device=DEV)
    q = torch.randn(2, 4, 64, device=DEV)
    lens = torch.tensor(contexts, dtype=torch.int32, device=DEV)
    out = hip_paged_decode(q, kc, vc, tables, lens)
    assert torch.isfinite(out).all()
    expected = oracle_decode(q, kc, vc, tables, lens, 1 / 8)
    assert max_abs(out, expected) <= 1e-5
    # Out-of-range ids are never dereferenced: those rows drop out of the softmax.
    bad = torch.tensor([[5, 1000, -1, -1], [0, 7, -7, -1]], dtype=torch.int32, device=DEV)
    out = hip_paged_decode(q, kc, vc, bad, lens)
    assert torch.isfinite(out).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("split_k", [None, 1])
def test_mfma_decode_never_uses_nan_slots(dtype, split_k):
    """16 Q / 8 KV heads, head_dim 128, 16-bit caches: the MFMA kernel reads
    whole 16-row tiles, so slots past each context (NaN here, as in an
    uninitialised pool) reach the tile; their weights are 0 and their V rows
    are zeroed before P.V, so the output matches the oracle, which like the
    reference's masked loads never reads them."""
    torch.manual_seed(6)
    kc = torch.full((64, 16, 8, 128), float("nan"), device=DEV).to(dtype)
    vc = kc.clone()
    contexts = [20, 33, 1, 16, 100, 47]
    tables = torch.full((len(contexts), 8), -1, dtype=torch.int32, device=DEV)
    ids = torch.randperm(63, device=DEV)[:sum((c + 15) // 16 for c in contexts)] + 1
    used = 0
    for r, c in enumerate(contexts):
        n = (c + 15) // 16
        tables[r, :n] = ids[used:used + n].int()
        used += n
        for pos in range(c):
            blk = int(tables[r, pos // 16])
            kc[blk, pos % 16] = torch.randn(8, 128, device=DEV).to(dtype)
            vc[blk, pos % 16] = torch.randn(8, 128, device=DEV).to(dtype)
    q = torch.randn(len(contexts), 16, 128, device=DEV).to(dtype)
    lens = torch.tensor(contexts, dtype=torch.int32, device=DEV)
    out = hip_paged_decode(q, kc, vc, tables, lens, split_k=split_k)
    assert torch.isfinite(out).all()
    expected = oracle_decode(q, kc, vc, tables, lens, 1 / math.sqrt(128))
    assert max_abs(out, expected) <= TOLERANCE[dtype]
    # Invalid ids read block 0 (all NaN) and drop out of the softmax.
    bad = tables.clone()
    bad[4, 1] = -1
    bad[5, 0] = 10 ** 6
    out = hip_paged_decode(q, kc, vc, bad, lens, split_k=split_k)
    assert torch.isfinite(out).all()


def test_split_counters_are_left_zeroed():
    from microinfer_amd.layer import hip_paged_attention as ops

    torch.manual_seed(6)
    kc = torch.randn(300, 16, 8, 128, device=DEV).to(torch.bfloat16)
    vc = torch.randn_like(kc)
    q = torch.randn(3, 32, 128, device=DEV).to(torch.bfloat16)
    tables = torch.randperm(300, device=DEV)[:300].reshape(3, 100).to(torch.int32)
    lens = torch.tensor([1600, 7, 900], dtype=torch.int32, device=DEV)
    first = hip_paged_decode(q, kc, vc, tables, lens, split_k=16)
    second = hip_paged_decode(q, kc, vc, tables, lens, split_k=16)
    third = hip_paged_decode(q, kc, vc, tables, lens)
    torch.cuda.synchronize()
    assert torch.equal(first, second)
    for counters in ops._counters.values():
        assert int(counters.abs().sum()) == 0
    expected = oracle_decode(q, kc, vc, tables, lens, 1 / math.sqrt(128))
    assert max_abs(first, expected) <= 2e-2 and max_abs(third, expected) <= 2e-2


@pytest.mark.parametrize("split_k", [None, 1, 4])
def test_shared_step_plan_matches_per_call_plan(split_k):
    from microinfer_amd.layer.hip_paged_attention import decode_plan

    torch.manual_seed(7)
    kc = torch.randn(2048, 16, 8, 128, device=DEV).to(torch.bfloat16)
    vc = torch.randn_like(kc)
    batch = make_decode_batch(num_seqs=24, ctx_lo=1, ctx_hi=1500, pool_blocks=2048,
                              draw_pools=False, **QWEN3_06B)
    tables = torch.tensor(batch.block_tables, device=DEV)
    lens = torch.tensor(batch.context_lens, device=DEV)
    plan = decode_plan(lens, num_kv_heads=8, block_size=16, block_table_width=tables.shape[1],
                       split_k=split_k)
    for layer in range(3):
        q = torch.randn(24, 16, 128, device=DEV).to(torch.bfloat16)
        own = hip_paged_decode(q, kc, vc, tables, lens, split_k=split_k)
        shared = hip_paged_decode(q, kc, vc, tables, lens, split_k=split_k, plan=plan)
        assert torch.equal(own, shared), f"layer {layer}"
    expected = oracle_decode(q, kc, vc, tables, lens, 1 / math.sqrt(128))
    assert max_abs(shared, expected) <= 2e-2


def test_hipgraph_replay_tracks_new_contexts():
    torch.manual_seed(5)
    kc = torch.randn(512, 16, 8, 128, device=DEV).to(torch.bfloat16)
    vc = torch.randn_like(kc)
    q = torch.randn(4, 16, 128, device=DEV).to(torch.bfloat16)
    tables = torch.randperm(512, device=DEV)[: 4 * 128].reshape(4, 128).to(torch.int32)
    lens = torch.tensor([10, 500, 1000, 2000], dtype=torch.int32, device=DEV)
    out = torch.empty_like(q)
    hip_paged_decode(q, kc, vc, tables, lens)  # warm-up outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with capture_graph(graph):
        out.copy_(hip_paged_decode(q, kc, vc, tables, lens))
    for step, new in enumerate([[11, 501, 1001, 2001], [1, 2048, 17, 300], [700, 700, 700, 700]]):
        lens.copy_(torch.tensor(new, dtype=torch.int32))
        q.normal_()
        graph.replay()
        torch.cuda.synchronize()
        eager = hip_paged_decode(q, kc, vc, tables, lens)
        assert torch.equal(out, eager), f"replay {step} differs from eager"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("hq,hkv,d", [(16, 8, 128), (8, 4, 64), (4, 1, 128)])
def test_many_sequences_take_half_width_groups(dtype, hq, hkv, d):
    # More (sequence, KV head) pairs than the device has CUs: the launch runs
    # two workgroups per CU (one ring slot per wave). Adaptive and forced
    # splits, and the fused append, must still match the oracle.
    rng = np.random.default_rng(11)
    num_seqs, bs = 300 // hkv + 40, 16
    contexts = rng.integers(1, 400, num_seqs)
    contexts[3], contexts[7], contexts[-1] = 0, 1, 2500
    width = int(-(-contexts.max() // bs))
    pool = int(sum(-(-c // bs) for c in contexts)) + 8
    perm = rng.permutation(pool)
    tables = np.full((num_seqs, width), -1, dtype=np.int32)
    used = 0
    for r, c in enumerate(contexts):
        n = int(-(-c // bs))
        tables[r, :n] = perm[used:used + n]
        used += n
    torch.manual_seed(12)
    kc = torch.randn(pool, bs, hkv, d, device=DEV).to(dtype)
    vc = torch.randn_like(kc)
    q = torch.randn(num_seqs, hq, d, device=DEV).to(dtype)
    t = torch.tensor(tables, device=DEV)
    lens = torch.tensor(contexts, dtype=torch.int32, device=DEV)
    expected = oracle_decode(q, kc, vc, t, lens, 1 / math.sqrt(d))
    assert max_abs(hip_paged_decode(q, kc, vc, t, lens), expected) <= TOLERANCE[dtype]
    assert max_abs(hip_paged_decode(q, kc, vc, t, lens, split_k=4), expected) <= TOLERANCE[dtype]
    # Fused append of each sequence's last row == append, then attend.
    live = contexts > 0
    new_k = torch.randn(num_seqs, hkv, d, device=DEV).to(dtype)
    new_v = torch.randn_like(new_k)
    kc2, vc2 = kc.clone(), vc.clone()
    fused = hip_paged_decode(q, kc2, vc2, t, lens, new_keys=new_k, new_values=new_v)
    for r in np.flatnonzero(live):
        pos = int(contexts[r]) - 1
        blk = int(tables[r, pos // bs])
        kc[blk, pos % bs] = new_k[r]
        vc[blk, pos % bs] = new_v[r]
    assert torch.equal(kc2, kc) and torch.equal(vc2, vc)
    expected = oracle_decode(q, kc, vc, t, lens, 1 / math.sqrt(d))
    assert max_abs(fused, expected) <= TOLERANCE[dtype]

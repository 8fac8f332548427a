"""Decode with the KV append fused into the attention launch.

The fused call must leave the caches bit-identical to an append of the same
rows at slot table[(c-1)//B]*B + (c-1)%B (the runner's decode slot,
microinfer/runner.py:167-174) and return the attention that append-then-
attend gives (microinfer/layer/cached_attention.py:76-85), within the
decode tolerances: 2e-3 fp32 / 2e-2 bf16 max-abs against the fp32 oracle.
"""

import math

import numpy as np
import pytest
import torch

from microinfer_amd.layer.hip_paged_attention import decode_plan, hip_paged_decode
from microinfer_amd.runner import capture_graph
from microinfer_amd.worker.kv_cache import KVCache
from microinfer_amd.workloads import QWEN3_06B, QWEN3_8B, make_decode_batch
from oracle import kv_append
from tests.support import TOLERANCE, bits, max_abs, oracle_decode, rounded

pytestmark = pytest.mark.gpu
DEV = "cuda"


def decode_slots(tables: np.ndarray, contexts, block_size: int) -> np.ndarray:
    return np.array([tables[r, (c - 1) // block_size] * block_size + (c - 1) % block_size
                     if c >= 1 else -1 for r, c in enumerate(contexts)], dtype=np.int64)


@pytest.mark.parametrize("split_k", [None, 1, 4, 64])
@pytest.mark.parametrize("layout", ["paired", "head_major", "token_major"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_fused_append_matches_append_then_attend(dtype, layout, split_k):
    batch = make_decode_batch(num_seqs=8, ctx_lo=1, ctx_hi=700, pool_blocks=1024, **QWEN3_06B)
    cache = KVCache(1, 1024, 16, 8, 128, dtype=dtype, device=DEV, layout=layout)
    cache.keys[0].copy_(rounded(batch.key_pool, dtype, DEV))
    cache.values[0].copy_(rounded(batch.value_pool, dtype, DEV))
    view = cache.layer(0)
    new_k = rounded(batch.new_keys, dtype, DEV)
    new_v = rounded(batch.new_values, dtype, DEV)
    expected_k, expected_v = bits(view.keys), bits(view.values)
    kv_append(expected_k, expected_v, batch.slots, bits(new_k), bits(new_v))

    q = rounded(batch.query, dtype, DEV)
    tables = torch.tensor(batch.block_tables, device=DEV)
    lens = torch.tensor(batch.context_lens, device=DEV)
    scale = 1 / math.sqrt(128)
    out = hip_paged_decode(q, view.keys, view.values, tables, lens, scale=scale, split_k=split_k,
                           new_keys=new_k, new_values=new_v)
    assert np.array_equal(bits(view.keys), expected_k)
    assert np.array_equal(bits(view.values), expected_v)
    expected = oracle_decode(q, view.keys, view.values, tables, lens, scale)
    assert max_abs(out, expected) <= TOLERANCE[dtype]


@pytest.mark.parametrize("num_seqs,lo,hi", [(32, 128, 2048), (4, 16384, 16384)])
def test_fused_append_at_workload_sizes(num_seqs, lo, hi):
    shape = QWEN3_06B if num_seqs == 32 else QWEN3_8B
    pool = 16384 if num_seqs == 32 else 65536
    hq, hkv = shape["num_q_heads"], shape["num_kv_heads"]
    batch = make_decode_batch(num_seqs=num_seqs, ctx_lo=lo, ctx_hi=hi, pool_blocks=pool,
                              draw_pools=False, **shape)
    cache = KVCache(1, pool, 16, hkv, 128, dtype=torch.bfloat16, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(0)
    cache.keys[0].copy_(torch.randn(cache.keys[0].shape, generator=gen, device=DEV))
    cache.values[0].copy_(torch.randn(cache.values[0].shape, generator=gen, device=DEV))
    view = cache.layer(0)
    q = rounded(batch.query, torch.bfloat16, DEV)
    new_k = torch.randn((num_seqs, hkv, 128), generator=gen, device=DEV).to(torch.bfloat16)
    new_v = torch.randn((num_seqs, hkv, 128), generator=gen, device=DEV).to(torch.bfloat16)
    tables = torch.tensor(batch.block_tables, device=DEV)
    lens = torch.tensor(batch.context_lens, device=DEV)
    slots = torch.tensor(decode_slots(batch.block_tables, batch.context_lens, 16), device=DEV)
    # Unfused order on a copy of the caches, fused call on the cache.
    ref_k, ref_v = view.keys.clone(), view.values.clone()
    ref_k[slots // 16, slots % 16] = new_k
    ref_v[slots // 16, slots % 16] = new_v
    out = hip_paged_decode(q, view.keys, view.values, tables, lens, new_keys=new_k,
                           new_values=new_v)
    assert torch.equal(view.keys, ref_k) and torch.equal(view.values, ref_v)
    del ref_k, ref_v
    unfused = hip_paged_decode(q, view.keys, view.values, tables, lens)
    assert float((out.float() - unfused.float()).abs().max()) <= 2e-2
    expected = oracle_decode(q, view.keys, view.values, tables, lens, 1 / math.sqrt(128))
    assert max_abs(out, expected) <= 2e-2


def test_fused_append_edge_cases():
    torch.manual_seed(11)
    hq, hkv, d = 8, 2, 64
    kc = torch.randn(12, 16, hkv, d, device=DEV)
    vc = torch.randn_like(kc)
    # ctx 0 (no append, zeros), ctx 1, a block boundary (16, 17), an invalid
    # block id at the append position (-1 and out of range), a valid context.
    contexts = [0, 1, 16, 17, 20, 33, 40]
    # Rows 4 and 5 append into block ids -1 and 1000 (pool of 12 blocks).
    # Row 6 shares blocks 2 and 0 with row 0, which appends nothing: a block
    # that receives a new row is never read by another sequence of the step.
    tables = torch.tensor([[0, 1, 2], [3, -1, -1], [4, 5, -1], [6, 7, -1], [8, -1, -1],
                           [9, 10, 1000], [11, 2, 0]], dtype=torch.int32, device=DEV)
    q = torch.randn(7, hq, d, device=DEV)
    new_k = torch.randn(7, hkv, d, device=DEV)
    new_v = torch.randn(7, hkv, d, device=DEV)
    lens = torch.tensor(contexts, dtype=torch.int32, device=DEV)

    slots = decode_slots(tables.cpu().numpy(), contexts, 16)
    host_k, host_v = kc.cpu().numpy().copy(), vc.cpu().numpy().copy()
    for r, s in enumerate(slots):
        if 0 <= s < 12 * 16:
            host_k[s // 16, s % 16] = new_k[r].cpu().numpy()
            host_v[s // 16, s % 16] = new_v[r].cpu().numpy()

    out = hip_paged_decode(q, kc, vc, tables, lens, new_keys=new_k, new_values=new_v)
    assert np.array_equal(bits(kc), bits(torch.from_numpy(host_k)))
    assert np.array_equal(bits(vc), bits(torch.from_numpy(host_v)))
    assert (out[0] == 0).all()
    assert torch.allclose(out[1], new_v[1].repeat_interleave(hq // hkv, dim=0), atol=1e-6)
    # Same result as the separate append (which skips the invalid slots)
    # followed by decode (which masks the invalid block ids).
    unfused = hip_paged_decode(q, kc, vc, tables, lens)
    assert float((out - unfused).abs().max()) <= 1e-5
    assert torch.isfinite(out).all()


def test_fused_append_reuses_plan_across_layers_and_graph_replay():
    torch.manual_seed(12)
    layers, seqs = 3, 6
    kcs = [torch.randn(512, 16, 8, 128, device=DEV).to(torch.bfloat16) for _ in range(layers)]
    vcs = [torch.randn_like(k) for k in kcs]
    tables = torch.randperm(512, device=DEV)[: seqs * 48].reshape(seqs, 48).to(torch.int32)
    lens = torch.tensor([5, 100, 300, 640, 17, 33], dtype=torch.int32, device=DEV)
    q = torch.randn(layers, seqs, 16, 128, device=DEV).to(torch.bfloat16)
    nk = torch.randn(layers, seqs, 8, 128, device=DEV).to(torch.bfloat16)
    nv = torch.randn_like(nk)
    outs = [torch.empty(seqs, 16, 128, device=DEV, dtype=torch.bfloat16) for _ in range(layers)]

    def step():
        plan = decode_plan(lens, num_kv_heads=8, block_size=16, block_table_width=48)
        for layer in range(layers):
            outs[layer].copy_(hip_paged_decode(q[layer], kcs[layer], vcs[layer], tables, lens,
                                               plan=plan, new_keys=nk[layer],
                                               new_values=nv[layer]))

    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with capture_graph(graph):
        step()
    for replay, new in enumerate([[6, 101, 301, 641, 18, 34], [7, 102, 302, 642, 19, 35]]):
        lens.copy_(torch.tensor(new, dtype=torch.int32))
        q.normal_()
        nk.normal_()
        nv.normal_()
        graph.replay()
        torch.cuda.synchronize()
        for layer in range(layers):
            for r, c in enumerate(new):
                blk, off = int(tables[r, (c - 1) // 16]), (c - 1) % 16
                assert torch.equal(kcs[layer][blk, off], nk[layer, r]), (replay, layer, r)
                assert torch.equal(vcs[layer][blk, off], nv[layer, r]), (replay, layer, r)
            expected = oracle_decode(q[layer], kcs[layer], vcs[layer], tables, lens,
                                     1 / math.sqrt(128))
            assert max_abs(outs[layer], expected) <= 2e-2, (replay, layer)


def test_fused_append_argument_errors():
    kc = torch.randn(4, 16, 2, 32, device=DEV)
    vc = torch.randn_like(kc)
    q = torch.randn(2, 4, 32, device=DEV)
    tables = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32, device=DEV)
    lens = torch.tensor([3, 20], dtype=torch.int32, device=DEV)
    rows = torch.randn(2, 2, 32, device=DEV)
    with pytest.raises(ValueError):
        hip_paged_decode(q, kc, vc, tables, lens, new_keys=rows)
    with pytest.raises(ValueError):
        hip_paged_decode(q, kc, vc, tables, lens, new_keys=rows[:1], new_values=rows[:1])
    with pytest.raises(ValueError):
        hip_paged_decode(q, kc, vc, tables, lens, new_keys=rows.half(), new_values=rows.half())
    with pytest.raises(ValueError):  # caches with different strides cannot be written in place
        hip_paged_decode(q, kc, vc.transpose(1, 2).contiguous().transpose(1, 2), tables, lens,
                         new_keys=rows, new_values=rows)

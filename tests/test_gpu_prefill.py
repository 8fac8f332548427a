"""Paged varlen (chunked prefill / mixed) attention on the GPU against the oracle.

Restates tests/layers/test_triton_paged_attention.py:80-145 (prefill vs the
reference path), tests/components/test_paged_attention.py:10-46 and :106-162
(dense-loop GQA and the small-block gather+varlen case), then the mixed
8B-shape workload: 8 chunks of 512 on shared-prefix caches plus 24 decode
rows in one launch, and the no-prefix (contiguous K/V) mode.
"""

import math

import numpy as np
import pytest
import torch

from microinfer_amd.layer.hip_paged_attention import hip_paged_prefill
from microinfer_amd.workloads import QWEN3_8B, make_mixed_prefill_batch
from oracle import dense_causal_attention_f64
from tests.support import (
    TOLERANCE,
    as_f32,
    checked_paged_attention,
    max_abs,
    oracle_attention,
    oracle_prefill,
)

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("block_size", [16, 64])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_prefill_matches_reference_small(block_size, dtype):
    torch.manual_seed(0)
    hq, hkv, d = 4, 2, 32
    contexts = [block_size + 5, 2 * block_size + 9]
    q_lens = [19, 7]
    max_blocks = max((c + block_size - 1) // block_size for c in contexts)
    tables = torch.arange(2 * max_blocks, dtype=torch.int32, device=DEV)
    tables = tables.reshape(2, max_blocks).flip(-1).contiguous()
    kc = torch.randn(2 * max_blocks, block_size, hkv, d, device=DEV, dtype=dtype)
    vc = torch.randn_like(kc)
    q = torch.randn(sum(q_lens), hq, d, device=DEV, dtype=dtype)
    cu_q = [0, 19, 26]
    cu_k = [0, contexts[0], sum(contexts)]
    scale = 1 / d**0.5
    expected = oracle_attention(q, kc, vc, tables, contexts, cu_q, scale)
    actual = hip_paged_prefill(q, kc, vc, torch.tensor(cu_q, device=DEV),
                               torch.tensor(cu_k, device=DEV), tables, max_seqlen_q=19,
                               scale=scale)
    assert actual.dtype == dtype
    assert max_abs(actual, expected) <= (1e-5 if dtype == torch.float32 else 2e-2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("prefix,query_len", [(0, 3), (2, 1), (1, 2)])
def test_paged_causal_gqa_matches_dense_loop(prefix, query_len, dtype):
    # test_paged_attention.py:10-46 on the device: physical order [2, 0].
    g = torch.Generator().manual_seed(0)
    context = prefix + query_len
    q = torch.randn(query_len, 4, 4, generator=g).to(dtype)
    lk = torch.randn(context, 2, 4, generator=g).to(dtype)
    lv = torch.randn(context, 2, 4, generator=g).to(dtype)
    k = torch.full((3, 2, 2, 4), 1000.0).to(dtype)
    v = torch.full_like(k, -1000)
    table = [2, 0]
    for pos in range(context):
        k[table[pos // 2], pos % 2] = lk[pos]
        v[table[pos // 2], pos % 2] = lv[pos]
    expected = dense_causal_attention_f64(q.float().numpy(), lk.float().numpy(), lv.float().numpy(),
                                          scale=0.5, prefix=prefix)
    actual = checked_paged_attention(
        q.to(DEV), k.to(DEV), v.to(DEV), torch.tensor([table], device=DEV),
        torch.tensor([context], device=DEV), torch.tensor([0, query_len], device=DEV),
    )
    assert actual.dtype == dtype and torch.isfinite(actual).all()
    tolerance = 1e-5 if dtype == torch.float32 else 1e-2
    np.testing.assert_allclose(as_f32(actual), expected, atol=tolerance, rtol=tolerance)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_small_block_prefill_with_prefix_reuse(dtype):
    # test_paged_attention.py:106-162: B=16, GQA 8/2, d=32, contexts [33, 17],
    # q_lens [16, 5], shuffled tables, poison +-1000 in unused slots.
    torch.manual_seed(0)
    bs, nblocks, hq, hkv, d = 16, 6, 8, 2, 32
    contexts, q_lens = [33, 17], [16, 5]
    tables = torch.tensor([[5, 1, 3], [0, 4, 2]], dtype=torch.int32, device=DEV)
    keys = torch.full((nblocks, bs, hkv, d), 1000.0, dtype=dtype, device=DEV)
    values = torch.full_like(keys, -1000.0)
    lk = torch.randn(sum(contexts), hkv, d, dtype=dtype, device=DEV)
    lv = torch.randn_like(lk)
    base = 0
    for r, c in enumerate(contexts):
        for t in range(c):
            blk = tables[r, t // bs]
            keys[blk, t % bs] = lk[base + t]
            values[blk, t % bs] = lv[base + t]
        base += c
    q = torch.randn(sum(q_lens), hq, d, dtype=dtype, device=DEV)
    scale = 1 / d**0.5
    expected = oracle_attention(q, keys, values, tables, contexts, [0, 16, 21], scale)
    actual = checked_paged_attention(q, keys, values, tables,
                                     torch.tensor(contexts, dtype=torch.int32, device=DEV),
                                     torch.tensor([0, 16, 21], dtype=torch.int32, device=DEV),
                                     scale=scale)
    assert max_abs(actual, expected) <= 2e-2


def _mixed_caches(batch, dtype):
    gen = torch.Generator(device=DEV).manual_seed(0)
    shape = (batch.pool_blocks, batch.block_size, 8, 128)
    kc = torch.randn(shape, generator=gen, device=DEV).to(dtype)
    vc = torch.randn(shape, generator=gen, device=DEV).to(dtype)
    return kc, vc


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_mixed_chunked_prefill_workload(dtype):
    # 8B shape: 8 prefill chunks of 512 on prefixes U[0, 3072] (first 1024
    # tokens shared), plus 24 decode rows with contexts U[256, 2048].
    batch = make_mixed_prefill_batch(pool_blocks=8192)
    kc, vc = _mixed_caches(batch, dtype)
    rng = np.random.default_rng(7)
    q = torch.from_numpy(rng.standard_normal((int(batch.q_lens.sum()), 32, 128),
                                             dtype=np.float32)).to(dtype).to(DEV)
    tables = torch.tensor(batch.block_tables, device=DEV)
    scale = 1 / math.sqrt(128)
    out = hip_paged_prefill(q, kc, vc, torch.tensor(batch.cu_seqlens_q, device=DEV),
                            torch.tensor(batch.cu_seqlens_k, device=DEV), tables,
                            max_seqlen_q=int(batch.q_lens.max()), scale=scale)
    expected = oracle_prefill(q, kc, vc, tables, batch.context_lens, batch.cu_seqlens_q, scale)
    assert max_abs(out, expected) <= 2e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_contiguous_no_prefix_prefill(dtype):
    torch.manual_seed(3)
    q_lens = [7, 1, 40]
    total = sum(q_lens)
    q = torch.randn(total, 8, 64, device=DEV).to(dtype)
    k = torch.randn(total, 2, 64, device=DEV).to(dtype)
    v = torch.randn(total, 2, 64, device=DEV).to(dtype)
    cu = torch.tensor([0, 7, 8, 48], dtype=torch.int32, device=DEV)
    out = hip_paged_prefill(q, k, v, cu, cu, None, max_seqlen_q=40)
    expected = np.concatenate([
        dense_causal_attention_f64(as_f32(q[a:b]), as_f32(k[a:b]), as_f32(v[a:b]),
                                   scale=1 / 8)
        for a, b in [(0, 7), (7, 8), (8, 48)]
    ])
    assert max_abs(out, expected) <= TOLERANCE[dtype]

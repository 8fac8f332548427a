"""The reference's own paged-attention tests, through the reference's names.

Restates tests/layers/test_triton_paged_attention.py:14-145 with its imports
pointed at ``microinfer_amd.layer.triton_paged_attention`` (the module a
maintainer binds in place of the Triton one): the decode case for block
sizes 16-256 and fp32 / fp16 / bf16 (reversed physical blocks, head_dim 32),
and the prefill case for block sizes 16 and 64 in fp16 / bf16 (19 and 7
query rows over one- and two-block-plus prefixes, flipped tables). The
expected values come from the CPU oracle in place of
``_paged_attention_reference``; the tolerances are the reference test's
(1e-5 fp32, 2e-2 half). ``_gather_paged_kv`` is checked bit-exact against
direct indexing of the pool.
"""

import numpy as np
import pytest
import torch

from microinfer_amd.layer.paged_attention import _gather_paged_kv
from microinfer_amd.layer.triton_paged_attention import (
    HAS_TRITON,
    triton_paged_decode,
    triton_paged_prefill,
)
from tests.support import as_f32, oracle_attention

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("block_size", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_triton_paged_decode_matches_reference(block_size, dtype):
    assert HAS_TRITON
    torch.manual_seed(0)
    num_requests, num_q_heads, num_kv_heads, head_dim = 2, 4, 2, 32
    contexts = [5, block_size + 3]
    num_blocks = (max(contexts) + block_size - 1) // block_size
    physical = list(range(num_requests * num_blocks))[::-1]
    block_tables = torch.tensor([physical[:num_blocks], physical[num_blocks:2 * num_blocks]],
                                dtype=torch.int32, device=DEV)
    key_cache = torch.randn(num_requests * num_blocks, block_size, num_kv_heads, head_dim,
                            device=DEV, dtype=dtype)
    value_cache = torch.randn_like(key_cache)
    query = torch.randn(num_requests, num_q_heads, head_dim, device=DEV, dtype=dtype)
    scale = 1.0 / head_dim ** 0.5
    expected = oracle_attention(query, key_cache, value_cache, block_tables, contexts,
                                [0, 1, 2], scale)
    actual = triton_paged_decode(query, key_cache, value_cache, block_tables,
                                 torch.tensor(contexts, dtype=torch.int32, device=DEV),
                                 scale=scale)
    tolerance = 1e-5 if dtype == torch.float32 else 2e-2
    np.testing.assert_allclose(as_f32(actual), expected, atol=tolerance, rtol=tolerance)
    assert actual.dtype == dtype


@pytest.mark.parametrize("split_k", [1, 2, 4, 8])
def test_triton_paged_decode_split_k_cap(split_k):
    # An explicit split_k (the reference's stripe count) caps the partitions;
    # the result equals the unsplit one to fp32 rounding.
    torch.manual_seed(1)
    block_size, contexts = 16, [700, 33]
    nb = (max(contexts) + block_size - 1) // block_size
    tables = torch.arange(2 * nb, dtype=torch.int32, device=DEV).reshape(2, nb).flip(0)
    kc = torch.randn(2 * nb, block_size, 2, 64, device=DEV)
    vc = torch.randn_like(kc)
    q = torch.randn(2, 8, 64, device=DEV)
    lens = torch.tensor(contexts, dtype=torch.int32, device=DEV)
    expected = oracle_attention(q, kc, vc, tables, contexts, [0, 1, 2], 0.125)
    out = triton_paged_decode(q, kc, vc, tables, lens, scale=0.125, split_k=split_k)
    np.testing.assert_allclose(as_f32(out), expected, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("block_size", [16, 64])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_triton_paged_prefill_matches_reference(block_size, dtype):
    torch.manual_seed(0)
    num_q_heads, num_kv_heads, head_dim = 4, 2, 32
    contexts = [block_size + 5, 2 * block_size + 9]
    q_lens = [19, 7]
    requests = len(contexts)
    max_blocks = max((c + block_size - 1) // block_size for c in contexts)
    block_tables = torch.arange(requests * max_blocks, dtype=torch.int32, device=DEV)
    block_tables = block_tables.reshape(requests, max_blocks).flip(-1).contiguous()
    key_cache = torch.zeros(requests * max_blocks, block_size, num_kv_heads, head_dim,
                            device=DEV, dtype=dtype)
    value_cache = torch.zeros_like(key_cache)
    for request, context in enumerate(contexts):
        for position in range(context):
            block = int(block_tables[request, position // block_size])
            key_cache[block, position % block_size] = torch.randn(num_kv_heads, head_dim,
                                                                  device=DEV, dtype=dtype)
            value_cache[block, position % block_size] = torch.randn(num_kv_heads, head_dim,
                                                                    device=DEV, dtype=dtype)
    total_q = sum(q_lens)
    query = torch.randn(total_q, num_q_heads, head_dim, device=DEV, dtype=dtype)
    cu_q, cu_k = [0], [0]
    for q_len, context in zip(q_lens, contexts):
        cu_q.append(cu_q[-1] + q_len)
        cu_k.append(cu_k[-1] + context)
    scale = 1.0 / head_dim ** 0.5
    expected = oracle_attention(query, key_cache, value_cache, block_tables, contexts, cu_q,
                                scale)
    actual = triton_paged_prefill(query, key_cache, value_cache,
                                  torch.tensor(cu_q, dtype=torch.int32, device=DEV),
                                  torch.tensor(cu_k, dtype=torch.int32, device=DEV),
                                  block_tables, max_seqlen_q=max(q_lens), scale=scale)
    np.testing.assert_allclose(as_f32(actual), expected, atol=2e-2, rtol=2e-2)
    assert actual.dtype == dtype


def test_triton_paged_prefill_mfma_shape():
    # The reference names at the MFMA kernel's shape (head_dim 128, GQA 4):
    # a 100-row chunk on a 300-token prefix.
    torch.manual_seed(2)
    block_size, ctx, q_len = 16, 400, 100
    nb = ctx // block_size
    tables = torch.randperm(64, device=DEV)[:nb].to(torch.int32)[None]
    kc = torch.randn(64, block_size, 2, 128, device=DEV, dtype=torch.bfloat16)
    vc = torch.randn_like(kc)
    q = torch.randn(q_len, 8, 128, device=DEV, dtype=torch.bfloat16)
    cu_q = torch.tensor([0, q_len], dtype=torch.int32, device=DEV)
    cu_k = torch.tensor([0, ctx], dtype=torch.int32, device=DEV)
    expected = oracle_attention(q, kc, vc, tables, [ctx], [0, q_len], 128 ** -0.5)
    actual = triton_paged_prefill(q, kc, vc, cu_q, cu_k, tables, max_seqlen_q=q_len)
    np.testing.assert_allclose(as_f32(actual), expected, atol=2e-2, rtol=2e-2)


def test_gather_paged_kv_reference_name_is_bit_exact():
    torch.manual_seed(3)
    block_size = 16
    kc = torch.randn(40, block_size, 2, 64, device=DEV, dtype=torch.bfloat16)
    vc = torch.randn_like(kc)
    tables = torch.randperm(40, device=DEV).to(torch.int32).reshape(4, 10)
    contexts = [1, 17, 160, 0]
    keys, values = _gather_paged_kv(kc, vc, tables, contexts, block_size)
    rows_k, rows_v = [], []
    for r, c in enumerate(contexts):
        for p in range(c):
            b = int(tables[r, p // block_size])
            rows_k.append(kc[b, p % block_size])
            rows_v.append(vc[b, p % block_size])
    assert torch.equal(keys, torch.stack(rows_k)) and torch.equal(values, torch.stack(rows_v))

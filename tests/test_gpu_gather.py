"""Block-table gather on the GPU: bit-exact against the oracle.

Restates the contract of ``_gather_paged_kv`` (microinfer/layer/paged_attention.py:76-101)
and tests/support/kv.py: each request's first c_r rows in logical order,
requests concatenated; shared prefix blocks, empty requests, both layouts.
"""

import numpy as np
import pytest
import torch

from microinfer_amd.layer.hip_paged_attention import hip_gather_kv
from microinfer_amd.layer.paged_attention import gather_paged_kv
from microinfer_amd.workloads import make_mixed_prefill_batch
from microinfer_amd.worker.kv_cache import KVCache
from oracle import gather_paged_kv as oracle_gather
from tests.support import bits

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("layout", ["paired", "head_major", "token_major"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_gather_small_bit_exact(layout, dtype):
    torch.manual_seed(0)
    cache = KVCache(1, 6, 4, 2, 8, dtype=dtype, device=DEV, layout=layout)
    cache.keys[0].copy_(torch.randn(6, 4, 2, 8, device=DEV))
    cache.values[0].copy_(torch.randn(6, 4, 2, 8, device=DEV))
    tables = torch.tensor([[5, 1, 3], [0, 4, -1], [2, -1, -1]], dtype=torch.int32, device=DEV)
    contexts = [9, 0, 4]
    k, v = gather_paged_kv(cache.keys[0], cache.values[0], tables, contexts, 4)
    ek, ev = oracle_gather(bits(cache.keys[0]), bits(cache.values[0]), tables.cpu().numpy(),
                           contexts, 4)
    assert np.array_equal(bits(k), ek) and np.array_equal(bits(v), ev)


def test_gather_mixed_workload_with_shared_prefix():
    batch = make_mixed_prefill_batch(pool_blocks=8192)
    cache = KVCache(1, 8192, 16, 8, 128, dtype=torch.bfloat16, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(1)
    cache.keys[0].copy_(torch.randn(cache.keys[0].shape, generator=gen, device=DEV))
    cache.values[0].copy_(torch.randn(cache.values[0].shape, generator=gen, device=DEV))
    tables = torch.tensor(batch.block_tables, device=DEV)
    contexts = [int(c) for c in batch.context_lens]
    k, v = gather_paged_kv(cache.keys[0], cache.values[0], tables, contexts, 16)
    assert k.shape == (sum(contexts), 8, 128)
    # Compare per request on the device (the pool is large).
    start = 0
    for r, c in enumerate(contexts):
        ids = tables[r, : (c + 15) // 16].long()
        rows_k = cache.keys[0][ids].reshape(-1, 8, 128)[:c]
        rows_v = cache.values[0][ids].reshape(-1, 8, 128)[:c]
        assert torch.equal(k[start : start + c], rows_k)
        assert torch.equal(v[start : start + c], rows_v)
        start += c


@pytest.mark.parametrize(
    "heads,head_dim,dtype",
    [
        (8, 128, torch.float32),   # 4 KiB rows: four 16-byte words per lane
        (16, 128, torch.float32),  # 8 KiB rows: the per-word kernel
        (8, 128, torch.bfloat16),  # two words per lane
        (1, 64, torch.bfloat16),   # one word per lane, most lanes idle
        (2, 4, torch.float16),     # 8-byte rows: 8-byte words
        (3, 2, torch.float16),     # 4-byte head rows
    ],
)
def test_gather_row_shapes_bit_exact(heads, head_dim, dtype):
    torch.manual_seed(3)
    cache = KVCache(1, 12, 16, heads, head_dim, dtype=dtype, device=DEV)
    cache.keys[0].copy_(torch.randn(cache.keys[0].shape, device=DEV))
    cache.values[0].copy_(torch.randn(cache.values[0].shape, device=DEV))
    tables = torch.tensor([[7, 2, 11, 0], [5, 9, -1, -1], [1, 3, 4, 6], [8, 10, -1, -1]],
                          dtype=torch.int32, device=DEV)
    contexts = [50, 17, 64, 1]
    k, v = gather_paged_kv(cache.keys[0], cache.values[0], tables, contexts, 16)
    ek, ev = oracle_gather(bits(cache.keys[0]), bits(cache.values[0]), tables.cpu().numpy(),
                           contexts, 16)
    assert np.array_equal(bits(k), ek) and np.array_equal(bits(v), ev)


def test_gather_rows_before_the_first_offset_read_as_zeros():
    # A cu_seqlens_k whose first entry is above zero: rows before it belong
    # to no request and come out as zeros (no table read before the row).
    cache = KVCache(1, 4, 16, 8, 128, dtype=torch.bfloat16, device=DEV)
    cache.keys[0].copy_(torch.randn(cache.keys[0].shape, device=DEV))
    cache.values[0].copy_(torch.randn(cache.values[0].shape, device=DEV))
    tables = torch.tensor([[2, 0]], dtype=torch.int32, device=DEV)
    cu = torch.tensor([3, 20], dtype=torch.int32, device=DEV)
    k, v = hip_gather_kv(cache.keys[0], cache.values[0], tables, cu, 20)
    assert not k[:3].any() and not v[:3].any()
    rows_k = cache.keys[0][tables[0].long()].reshape(-1, 8, 128)[:17]
    rows_v = cache.values[0][tables[0].long()].reshape(-1, 8, 128)[:17]
    assert torch.equal(k[3:], rows_k) and torch.equal(v[3:], rows_v)


def test_gather_rejects_short_tables():
    cache = KVCache(1, 2, 4, 1, 8, device=DEV)
    with pytest.raises(ValueError):
        gather_paged_kv(cache.keys[0], cache.values[0],
                        torch.tensor([[0]], dtype=torch.int32, device=DEV), [5], 4)

"""Block-table gather on the GPU: bit-exact against the oracle.

Restates the contract of ``_gather_paged_kv`` (microinfer/layer/paged_attention.py:76-101)
and tests/support/kv.py: each request's first c_r rows in logical order,
requests concatenated; shared prefix blocks, empty requests, both layouts.
"""

import numpy as np
import pytest
import torch

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


def test_gather_rejects_short_tables():
    cache = KVCache(1, 2, 4, 1, 8, device=DEV)
    with pytest.raises(ValueError):
        gather_paged_kv(cache.keys[0], cache.values[0],
                        torch.tensor([[0]], dtype=torch.int32, device=DEV), [5], 4)

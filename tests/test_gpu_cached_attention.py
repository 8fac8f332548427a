"""CachedAttention on the GPU: append-then-attend through AttentionMetadata.

Restates tests/components/test_cache_binding.py:102-163: chunked prefill +
decode over non-contiguous physical blocks equals one dense causal pass, the
no-prefix prefill isolates packed requests, and the fast write path equals
the checked one.
"""

import pytest
import torch

from microinfer_amd.layer.cached_attention import CachedAttention
from microinfer_amd.layer.metadata import AttentionMetadata
from microinfer_amd.worker.kv_cache import KVCache

pytestmark = pytest.mark.gpu
DEV = "cuda"


def dense_reference(q, k, v):
    q, k, v = q.double().cpu(), k.double().cpu(), v.double().cpu()
    result = torch.empty_like(q)
    repeats = q.shape[1] // k.shape[1]
    for i in range(len(q)):
        for h in range(q.shape[1]):
            weights = (k[: i + 1, h // repeats] @ q[i, h] / q.shape[-1] ** 0.5).softmax(0)
            result[i, h] = weights @ v[: i + 1, h // repeats]
    return result.float()


@pytest.mark.parametrize("layout", ["paired", "head_major", "token_major"])
@pytest.mark.parametrize("checked", [True, False])
def test_chunks_and_decode_match_full_prefill(layout, checked, seeded_torch):
    q, k, v = torch.randn(6, 4, 4), torch.randn(6, 2, 4), torch.randn(6, 2, 4)
    expected = dense_reference(q, k, v)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    backend = CachedAttention()
    pool = KVCache(2, 4, 2, 2, 4, device=DEV, layout=layout)
    backend.bind_cache(pool.layer(1))
    slots = torch.tensor([4, 5, 0, 1, 6, 7], dtype=torch.int32, device=DEV)
    table = torch.tensor([[2, 0, 3]], dtype=torch.int32, device=DEV)
    outputs = []
    for start, end in [(0, 3), (3, 5), (5, 6)]:
        if start != 5:
            metadata = AttentionMetadata.build(
                is_prefill=True,
                cu_seqlens_q=torch.tensor([0, end - start], dtype=torch.int32, device=DEV),
                cu_seqlens_k=torch.tensor([0, end], dtype=torch.int32, device=DEV),
                max_seqlen_q=end - start,
                max_seqlen_k=end,
                slot_mapping=slots[start:end],
                block_tables=None if start == 0 else table,
                validate_cache_write=checked,
            )
        else:
            metadata = AttentionMetadata.build(
                is_prefill=False,
                slot_mapping=slots[start:end],
                context_lens=torch.tensor([end], dtype=torch.int32, device=DEV),
                block_tables=table,
                validate_cache_write=checked,
            )
        outputs.append(backend(q[start:end], k[start:end], v[start:end], metadata))
    torch.testing.assert_close(torch.cat(outputs).cpu(), expected, atol=1e-5, rtol=1e-5)
    assert pool.keys[0].eq(0).all()
    gathered = torch.cat([pool.keys[1, 2], pool.keys[1, 0], pool.keys[1, 3]])[:6]
    assert torch.equal(gathered, k)


def test_no_prefix_prefill_isolates_requests(seeded_torch):
    q, k, v = torch.randn(5, 4, 4), torch.randn(5, 2, 4), torch.randn(5, 2, 4)
    cu = torch.tensor([0, 3, 5], dtype=torch.int32, device=DEV)
    metadata = AttentionMetadata.build(is_prefill=True, cu_seqlens_q=cu, cu_seqlens_k=cu,
                                       max_seqlen_q=3, max_seqlen_k=5)
    actual = CachedAttention()(q.to(DEV), k.to(DEV), v.to(DEV), metadata)
    expected = torch.cat([dense_reference(q[:3], k[:3], v[:3]), dense_reference(q[3:], k[3:], v[3:])])
    torch.testing.assert_close(actual.cpu(), expected, atol=1e-5, rtol=1e-5)


def test_fast_cache_write_matches_checked_path(seeded_torch):
    q, k, v = torch.randn(3, 4, 4), torch.randn(3, 2, 4), torch.randn(3, 2, 4)
    pool = KVCache(1, 2, 4, 2, 4, device=DEV)
    backend = CachedAttention()
    backend.bind_cache(pool.layer(0))
    cu = torch.tensor([0, 3], dtype=torch.int32, device=DEV)
    metadata = AttentionMetadata.build(
        is_prefill=True, cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=3, max_seqlen_k=3,
        slot_mapping=torch.tensor([0, 1, 2], dtype=torch.int32, device=DEV),
        validate_cache_write=False,
    )
    actual = backend(q.to(DEV), k.to(DEV), v.to(DEV), metadata)
    torch.testing.assert_close(actual.cpu(), dense_reference(q, k, v), atol=1e-5, rtol=1e-5)
    assert torch.equal(pool.layer(0).keys[0, :3].cpu(), k)
    assert torch.equal(pool.layer(0).values[0, :3].cpu(), v)

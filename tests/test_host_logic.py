"""Host-side contracts that need no GPU: metadata, cache layout, validation.

Restates tests/components/test_metadata.py:11-57, the layout and atomic-write
parts of tests/components/test_kv_cache.py and test_cache_binding.py, and the
ValueError contracts of the reference's Triton wrappers. Anything that would
launch a kernel on CPU tensors must raise (there is no CPU fallback).
"""

import pytest
import torch

from microinfer_amd.layer.cached_attention import CachedAttention
from microinfer_amd.layer.hip_paged_attention import hip_paged_decode, hip_paged_prefill
from microinfer_amd.layer.metadata import AttentionMetadata
from microinfer_amd.layer.paged_attention import paged_attention_meta
from microinfer_amd.worker.hip_kv_store import store_kv
from microinfer_amd.worker.kv_cache import KVCache


def test_prefill_metadata_derives_lists_lazily():
    metadata = AttentionMetadata.build(
        is_prefill=True,
        cu_seqlens_q=torch.tensor([0, 2, 5], dtype=torch.int32),
        cu_seqlens_k=torch.tensor([0, 2, 5], dtype=torch.int32),
        max_seqlen_q=3,
        max_seqlen_k=5,
        slot_mapping=torch.tensor([0, 1, 2], dtype=torch.int32),
    )
    assert metadata.direct_prefill
    assert metadata.cu_q_cpu == (0, 2, 5)
    assert metadata.q_lens_cpu == (2, 3)
    assert metadata.context_lens_cpu == (2, 3)
    assert metadata.cu_q_cpu is metadata.cu_q_cpu


def test_decode_metadata_derives_query_offsets():
    metadata = AttentionMetadata.build(
        is_prefill=False,
        context_lens=torch.tensor([3, 4], dtype=torch.int32),
        slot_mapping=torch.tensor([2, 3], dtype=torch.int32),
        block_tables=torch.tensor([[0], [1]], dtype=torch.int32),
    )
    assert metadata.is_decode and not metadata.direct_prefill
    assert metadata.cu_q_cpu == (0, 1, 2)
    assert metadata.q_lens_cpu == (1, 1)
    assert metadata.context_lens_cpu == (3, 4)


def test_slot_indices_are_cached_per_block_size():
    metadata = AttentionMetadata.build(
        is_prefill=False, slot_mapping=torch.tensor([0, 5, 2], dtype=torch.int32)
    )
    blocks, offsets = metadata.slot_indices(4)
    assert blocks.tolist() == [0, 1, 0] and offsets.tolist() == [0, 1, 2]
    assert metadata.slot_indices(4)[0] is blocks
    assert metadata.slot_mapping_long.dtype == torch.long
    blocks2, offsets2 = metadata.slot_indices(2)
    assert blocks2.tolist() == [0, 2, 1] and offsets2.tolist() == [0, 1, 0]


@pytest.mark.parametrize("layout", ["paired", "head_major", "token_major"])
def test_cache_layout_byte_budget_and_views(layout):
    cache = KVCache(2, 3, 4, 2, 3, layout=layout)
    assert cache.keys.shape == cache.values.shape == (2, 3, 4, 2, 3)
    assert cache.num_bytes == 2 * 2 * 3 * 4 * 2 * 3 * 4
    view = cache.layer(1)
    assert view.keys.untyped_storage().data_ptr() == cache.keys.untyped_storage().data_ptr()
    assert view.block_size == 4
    if layout == "paired":
        # K then V of one KV head's block are one contiguous run: token
        # stride D, head stride 2*B*D, V one B*D after K, equal strides.
        assert view.keys.stride() == view.values.stride() == (2 * 2 * 4 * 3, 3, 2 * 4 * 3, 1)
        assert view.values.data_ptr() - view.keys.data_ptr() == 4 * 3 * 4
        cache.values[1, 2, 3, 1] = -5.0
        assert cache.keys[1, 2, 3, 1].eq(0).all()
        cache.values[1, 2, 3, 1] = 0.0
    elif layout == "head_major":
        # One KV head's block is contiguous: token stride D, head stride B*D.
        assert view.keys.stride() == (2 * 4 * 3, 3, 4 * 3, 1)
    else:
        assert view.keys.is_contiguous()
    cache.keys[1, 2, 3, 1] = 7.0
    assert view.keys[2, 3, 1].eq(7).all()
    with pytest.raises(ValueError):
        cache.layer(2)
    with pytest.raises(ValueError):
        KVCache(0, 1, 1, 1, 1)


@pytest.mark.parametrize("slots", [[0, 8], [0, -2], [0, 0]])
def test_invalid_checked_writes_are_atomic(slots):
    cache = KVCache(1, 2, 4, 1, 2)
    cache.keys.fill_(7)
    cache.values.fill_(7)
    with pytest.raises(ValueError):
        cache.layer(0).write_checked(torch.tensor(slots), torch.zeros(2, 1, 2), torch.zeros(2, 1, 2))
    assert (cache.keys == 7).all() and (cache.values == 7).all()


def test_checked_write_validates_both_inputs_first():
    view = KVCache(1, 1, 2, 1, 4).layer(0)
    with pytest.raises(ValueError):
        view.write_checked(torch.tensor([0]), torch.ones(1, 1, 4), torch.ones(2, 1, 4))
    assert view.keys.eq(0).all()


def test_writes_and_attention_refuse_cpu_tensors():
    view = KVCache(1, 2, 4, 1, 2).layer(0)
    with pytest.raises(RuntimeError, match="HIP device"):
        view.write_checked(torch.tensor([1]), torch.ones(1, 1, 2), torch.ones(1, 1, 2))
    with pytest.raises(RuntimeError, match="HIP device"):
        view.write_slots(torch.tensor([1], dtype=torch.int32), torch.ones(1, 1, 2), torch.ones(1, 1, 2))
    metadata = AttentionMetadata.build(
        is_prefill=False,
        context_lens=torch.tensor([1]),
        block_tables=torch.tensor([[0]]),
    )
    with pytest.raises(RuntimeError, match="HIP device"):
        paged_attention_meta(torch.zeros(1, 2, 2), view.keys, view.values, metadata)


def test_decode_without_bound_cache_fails_clearly():
    metadata = AttentionMetadata.build(
        is_prefill=False, context_lens=torch.tensor([1]), block_tables=torch.tensor([[0]])
    )
    q = torch.zeros(1, 1, 4)
    with pytest.raises(RuntimeError, match="bound layer cache"):
        CachedAttention()(q, q, q, metadata)


def test_wrapper_value_errors_mirror_reference():
    cache = torch.zeros(4, 16, 2, 32)
    with pytest.raises(ValueError, match="query must have shape"):
        hip_paged_decode(torch.zeros(2, 32), cache, cache, torch.zeros(2, 1), torch.zeros(2))
    with pytest.raises(ValueError, match="share device/dtype"):
        hip_paged_decode(torch.zeros(2, 4, 32, dtype=torch.float16), cache, cache,
                         torch.zeros(2, 1), torch.zeros(2))
    with pytest.raises(ValueError, match="GPU device"):
        hip_paged_decode(torch.zeros(2, 4, 32), cache, cache, torch.zeros(2, 1), torch.zeros(2))
    assert hip_paged_decode(torch.zeros(0, 4, 32), cache, cache, torch.zeros(0, 1),
                            torch.zeros(0)).shape == (0, 4, 32)
    with pytest.raises(ValueError, match="query must have shape"):
        hip_paged_prefill(torch.zeros(3, 32), cache, cache, torch.zeros(2), torch.zeros(2),
                          torch.zeros(1, 1), max_seqlen_q=3)
    with pytest.raises(ValueError, match="K/V shapes differ"):
        store_kv(cache, cache, torch.zeros(1), torch.zeros(1), torch.zeros(1, 2, 32),
                 torch.zeros(2, 2, 32), 16)
    with pytest.raises(ValueError, match="inner dimensions"):
        store_kv(cache, cache, torch.zeros(1), torch.zeros(1), torch.zeros(1, 32, 2).transpose(1, 2),
                 torch.zeros(1, 2, 32), 16)

"""KV append on the GPU: bit-exact against the oracle's scatter.

Covers the reference's append contracts (microinfer/worker/kv_cache.py:30-79,
triton_kv_store.py:45-78; tests/components/test_kv_cache.py): slot -> (block,
offset), -1 padding skipped, blocks/offsets form, fused-QKV strided inputs,
both cache layouts, every dtype, and the workload sizes of the decode configs.
"""

import numpy as np
import pytest
import torch

from microinfer_amd.workloads import QWEN3_06B, make_decode_batch
from microinfer_amd.worker.hip_kv_store import store_kv
from microinfer_amd.worker.kv_cache import KVCache
from oracle import kv_append
from tests.support import bits, rounded

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def filled_cache(batch, dtype, layout):
    n, b, h, d = batch.key_pool.shape
    cache = KVCache(1, n, b, h, d, dtype=dtype, device=DEV, layout=layout)
    cache.keys[0].copy_(rounded(batch.key_pool, dtype, DEV))
    cache.values[0].copy_(rounded(batch.value_pool, dtype, DEV))
    return cache


@pytest.mark.parametrize("layout", ["paired", "head_major", "token_major"])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("slot_dtype", [torch.int32, torch.int64])
def test_append_small_decode_workload_bit_exact(layout, dtype, slot_dtype):
    # 0.6B layer shape, pool 1024, 8 sequences, contexts U[64, 512], seed 0.
    batch = make_decode_batch(num_seqs=8, ctx_lo=64, ctx_hi=512, pool_blocks=1024, **QWEN3_06B)
    cache = filled_cache(batch, dtype, layout)
    view = cache.layer(0)
    expected_k, expected_v = bits(view.keys), bits(view.values)
    new_k = rounded(batch.new_keys, dtype, DEV)
    new_v = rounded(batch.new_values, dtype, DEV)
    view.write_slots(torch.tensor(batch.slots, dtype=slot_dtype, device=DEV), new_k, new_v)
    kv_append(expected_k, expected_v, batch.slots, bits(new_k), bits(new_v))
    assert np.array_equal(bits(view.keys), expected_k)
    assert np.array_equal(bits(view.values), expected_v)


@pytest.mark.parametrize("layout", ["paired", "head_major", "token_major"])
def test_append_full_decode_pool(layout):
    # 0.6B shape, bf16, pool 16384, 32 sequences, contexts U[128, 2048].
    batch = make_decode_batch(num_seqs=32, ctx_lo=128, ctx_hi=2048, pool_blocks=16384,
                              draw_pools=False, **QWEN3_06B)
    cache = KVCache(1, 16384, 16, 8, 128, dtype=torch.bfloat16, device=DEV, layout=layout)
    gen = torch.Generator(device=DEV).manual_seed(0)
    cache.keys[0].copy_(torch.randn(cache.keys[0].shape, generator=gen, device=DEV))
    cache.values[0].copy_(torch.randn(cache.values[0].shape, generator=gen, device=DEV))
    before_k, before_v = cache.keys[0].clone(), cache.values[0].clone()
    rng = np.random.default_rng(1)
    new_k = rounded(rng.standard_normal((32, 8, 128)), torch.bfloat16, DEV)
    new_v = rounded(rng.standard_normal((32, 8, 128)), torch.bfloat16, DEV)
    cache.layer(0).write_slots(torch.tensor(batch.slots, dtype=torch.int32, device=DEV), new_k, new_v)
    slots = torch.tensor(batch.slots, dtype=torch.long, device=DEV)
    blk, off = slots // 16, slots % 16
    assert torch.equal(cache.keys[0][blk, off], new_k)
    assert torch.equal(cache.values[0][blk, off], new_v)
    # Everything else is untouched.
    before_k[blk, off] = new_k
    before_v[blk, off] = new_v
    assert torch.equal(cache.keys[0], before_k) and torch.equal(cache.values[0], before_v)


def test_padding_and_block_offset_forms():
    cache = KVCache(1, 2, 4, 1, 2, device=DEV)
    cache.keys.fill_(9)
    cache.values.fill_(9)
    view = cache.layer(0)
    view.write_checked(torch.tensor([-1, 0], device=DEV), torch.zeros(2, 1, 2, device=DEV),
                       torch.ones(2, 1, 2, device=DEV))
    assert (cache.keys[0, 0, -1, -1] == 9).all() and (cache.keys[0, 1, -1, -1] == 9).all()
    assert (cache.keys[0, 0, 0, 0] == 0).all() and (cache.values[0, 0, 0, 0] == 1).all()
    fast = KVCache(1, 2, 4, 1, 2, device=DEV)
    checked = KVCache(1, 2, 4, 1, 2, device=DEV)
    keys = torch.randn(3, 1, 2, device=DEV)
    values = torch.randn(3, 1, 2, device=DEV)
    slots = torch.tensor([0, 5, 2], device=DEV)
    checked.layer(0).write_checked(slots, keys, values)
    fast.layer(0).write_fast(slots // 4, slots % 4, keys, values)
    assert torch.equal(checked.keys, fast.keys) and torch.equal(checked.values, fast.values)


def test_known_answer_roundtrip_on_device():
    # test_kv_cache.py:10-23.
    cache = KVCache(2, 3, 4, 2, 3, device=DEV)
    keys = torch.arange(30, dtype=torch.float32, device=DEV).reshape(5, 2, 3)
    cache.keys.fill_(-5)
    cache.values.fill_(-6)
    cache.layer(1).write_checked(torch.tensor([8, 9, 10, 11, 0], device=DEV), keys, keys + 100)
    view = cache.layer(1)
    rows = torch.cat([view.keys[2], view.keys[0]])[:5]
    assert torch.equal(rows, keys)
    assert torch.equal(torch.cat([view.values[2], view.values[0]])[:5], keys + 100)
    assert (cache.keys[0] == -5).all() and (cache.keys[1, 1] == -5).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fused_qkv_strided_rows(dtype):
    # K/V are column slices of a fused [T, (Hq + 2 Hkv) * D] projection.
    tokens, hq, hkv, d = 5, 4, 2, 64
    qkv = torch.randn(tokens, (hq + 2 * hkv) * d, device=DEV).to(dtype)
    k = qkv[:, hq * d : (hq + hkv) * d].view(tokens, hkv, d)
    v = qkv[:, (hq + hkv) * d :].view(tokens, hkv, d)
    assert not k.is_contiguous()
    cache = KVCache(1, 4, 16, hkv, d, dtype=dtype, device=DEV)
    slots = torch.tensor([3, 17, 40, 63, 0], device=DEV, dtype=torch.int32)
    cache.layer(0).write_slots(slots, k, v)
    s = slots.long()
    assert torch.equal(cache.keys[0][s // 16, s % 16], k)
    assert torch.equal(cache.values[0][s // 16, s % 16], v)


def test_store_kv_signature_and_duplicate_pad_slots():
    cache = KVCache(1, 3, 4, 2, 8, dtype=torch.bfloat16, device=DEV)
    keys = torch.randn(3, 2, 8, device=DEV).to(torch.bfloat16)
    blocks = torch.tensor([2, 2, 1], device=DEV)
    offsets = torch.tensor([1, 1, 3], device=DEV)
    store_kv(cache.keys[0], cache.values[0], blocks, offsets, keys, keys, 4)
    landed = cache.keys[0, 2, 1]
    assert torch.equal(landed, keys[0]) or torch.equal(landed, keys[1])
    assert torch.equal(cache.keys[0, 1, 3], keys[2])
    assert (cache.keys[0, 0] == 0).all()

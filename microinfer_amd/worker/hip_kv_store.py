"""KV-cache append through the HIP library.

Mirrors ``store_kv`` (microinfer/worker/triton_kv_store.py:45-78): same
signature, same ValueErrors, but one gfx950 kernel that also takes the slot
map directly, so the per-step ``slot // B`` / ``slot % B`` tensors
(microinfer/layer/metadata.py:75-84) are folded into the append.
"""

from __future__ import annotations

import torch

from microinfer_amd import _lib

_INDEX_DTYPES = (torch.int32, torch.int64)


def _cache_strides(key_cache: torch.Tensor, value_cache: torch.Tensor):
    if key_cache.ndim != 4 or key_cache.shape != value_cache.shape:
        raise ValueError("K/V caches must have matching [blocks, B, Hkv, D] shapes")
    if key_cache.stride() != value_cache.stride():
        raise ValueError("K/V caches must share one layout")
    if key_cache.stride(-1) != 1:
        raise ValueError("cache head_dim must be contiguous")
    return key_cache.stride(0), key_cache.stride(1), key_cache.stride(2)


def launch_append(key_cache, value_cache, index0, index1, keys, values) -> None:
    """Write ``keys``/``values [T, Hkv, D]`` into the caches on the GPU.

    ``index1 is None``: ``index0`` is the slot map (negative slots skipped).
    Otherwise ``index0``/``index1`` are block ids and in-block offsets.
    """
    _lib.require_device(key_cache, value_cache, index0, index1, keys, values,
                        what="KV append")
    if keys.ndim != 3 or values.shape != keys.shape:
        raise ValueError("K/V must have matching [tokens, Hkv, D] shapes")
    if keys.shape[1:] != key_cache.shape[2:]:
        raise ValueError("K/V heads must match the cache")
    if keys.dtype != key_cache.dtype or values.dtype != key_cache.dtype:
        raise ValueError("K/V dtype must match the cache")
    if keys.stride(-1) != 1:
        keys = keys.contiguous()
    if values.stride(-1) != 1:
        values = values.contiguous()
    if index0.dtype not in _INDEX_DTYPES:
        raise ValueError("slot indices must be int32 or int64")
    if index1 is not None and index1.dtype != index0.dtype:
        index1 = index1.to(index0.dtype)
    index0 = index0.contiguous()
    index1 = None if index1 is None else index1.contiguous()
    if index0.numel() != keys.shape[0] or (index1 is not None and index1.numel() != keys.shape[0]):
        raise ValueError("one slot per token is required")
    c_bs, c_ts, c_hs = _cache_strides(key_cache, value_cache)
    tokens, heads, head_dim = keys.shape
    if tokens == 0:
        return
    lib = _lib.load()
    status = lib.mi_kv_append(
        keys.data_ptr(), keys.stride(0), keys.stride(1),
        values.data_ptr(), values.stride(0), values.stride(1),
        key_cache.data_ptr(), value_cache.data_ptr(), c_bs, c_ts, c_hs,
        index0.data_ptr(), None if index1 is None else index1.data_ptr(),
        int(index0.dtype == torch.int64), tokens, heads, head_dim,
        key_cache.shape[1], key_cache.shape[0], _lib.dtype_code(key_cache.dtype),
        _lib.stream_handle(key_cache.device),
    )
    _lib.check(status, "mi_kv_append")


def store_kv(key_cache, value_cache, blocks, offsets, keys, values, block_size: int):
    """Signature and checks of the reference ``store_kv`` (triton_kv_store.py:45-63)."""
    _tokens, _heads, head_dim = keys.shape
    if values.shape != keys.shape:
        raise ValueError("K/V shapes differ")
    if keys.stride(-1) != 1 or keys.stride(-2) != head_dim:
        raise ValueError("K/V inner dimensions must be contiguous")
    if values.stride(-1) != 1 or values.stride(-2) != head_dim:
        raise ValueError("V inner dimensions must be contiguous")
    if block_size != key_cache.shape[1]:
        raise ValueError("block_size does not match the cache")
    launch_append(key_cache, value_cache, blocks, offsets, keys, values)


def append_slots(key_cache, value_cache, slot_mapping, keys, values) -> None:
    """Append with the raw slot map (``-1`` = padding), slot -> (block, offset) in-kernel."""
    launch_append(key_cache, value_cache, slot_mapping, None, keys, values)

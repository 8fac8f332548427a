"""Attention over one layer's KV cache, driven by AttentionMetadata.

Mirrors ``CachedAttention`` (microinfer/layer/cached_attention.py:56-101):
append this step's K/V first (checked or fast), then attend, so attention
sees the current tokens. The no-prefix prefill runs the same HIP varlen
kernel on the contiguous K/V instead of FlashAttention or an SDPA loop.
"""

from __future__ import annotations

from torch import nn

from microinfer_amd.layer.paged_attention import paged_attention_meta, varlen_attention
from microinfer_amd.worker.kv_cache import LayerKVCache


class CachedAttention(nn.Module):
    def __init__(self):
        super().__init__()
        self.cache: LayerKVCache | None = None

    def bind_cache(self, cache: LayerKVCache):
        self.cache = cache

    def forward(self, q, k, v, metadata):
        """Q/K already normalised and rotated. Returns ``[T, Hq, D]``."""
        cache = self.cache
        direct = metadata.direct_prefill if metadata.is_prefill else False
        if not direct and (cache is None or metadata.block_tables is None):
            raise RuntimeError("paged attention requires a bound layer cache and block table")
        if cache is not None:
            if metadata.slot_mapping is None:
                raise ValueError("bound cache requires slot_mapping")
            if metadata.validate_cache_write:
                cache.write_checked(metadata.slot_mapping, k, v)
            else:
                cache.write_slots(metadata.slot_mapping, k, v)
        if not direct:
            return paged_attention_meta(q, cache.keys, cache.values, metadata)
        if q.shape[1] % k.shape[1]:
            raise ValueError("query heads must be divisible by KV heads")
        return varlen_attention(q, k, v, metadata)

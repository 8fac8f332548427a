"""Attention-backend dispatcher over the HIP kernels.

Mirrors ``paged_attention_meta`` and ``_gather_paged_kv``
(microinfer/layer/paged_attention.py:188-293, :76-101). The reference picks
between FlashAttention, Triton, gather + FA varlen and its PyTorch reference;
here every route is a gfx950 kernel and nothing falls back to the CPU:

* decode metadata        -> ``hip_paged_decode`` (split-K planned on device)
* prefill / mixed chunks -> ``hip_paged_prefill`` (reads the pages in place,
  so the reference's ``Σctx >= 4 Σq`` choice between in-place and gathered
  prefill, :104-139, disappears)

``gather_paged_kv`` (also under the reference's name ``_gather_paged_kv``)
keeps the reference's signature for callers that need contiguous varlen K/V;
it is one launch instead of two ``index_select`` per request plus ``cat``.
"""

from __future__ import annotations

import math

import torch

from microinfer_amd.layer.hip_paged_attention import (
    hip_gather_kv,
    hip_paged_decode,
    hip_paged_prefill,
)
from microinfer_amd.layer.metadata import AttentionMetadata


def gather_paged_kv(key_cache, value_cache, block_tables, contexts, block_size):
    """Materialise each request's first ``contexts[r]`` rows as varlen K/V.

    Same arguments as ``_gather_paged_kv`` (paged_attention.py:76): host-side
    ``contexts``; returns ``(keys, values)`` of shape ``[sum(contexts), Hkv, D]``.
    """
    if block_size != key_cache.shape[1]:
        raise ValueError("block_size does not match the cache")
    contexts = [int(c) for c in contexts]
    if any(c < 0 for c in contexts):
        raise ValueError("contexts must be nonnegative")
    width = block_tables.shape[1]
    if any((c + block_size - 1) // block_size > width for c in contexts):
        raise ValueError("block table does not cover the context")
    offsets = [0]
    for length in contexts:
        offsets.append(offsets[-1] + length)
    cu_k = torch.tensor(offsets, dtype=torch.int32, device=key_cache.device)
    return hip_gather_kv(key_cache, value_cache, block_tables[: len(contexts)], cu_k, offsets[-1])


# The reference's name (paged_attention.py:76), for callers bound to it.
_gather_paged_kv = gather_paged_kv


def paged_attention_meta(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    metadata: AttentionMetadata,
    *,
    scale: float | None = None,
) -> torch.Tensor:
    """Kernel dispatch for validated metadata; no host validation or tolist."""
    if query.shape[0] == 0:
        return torch.empty_like(query)
    if scale is None:
        scale = 1.0 / math.sqrt(query.shape[-1])
    if not query.is_cuda:
        raise RuntimeError(
            "paged_attention_meta runs on the HIP device only; "
            f"got a {query.device} query"
        )
    if metadata.block_tables is None:
        raise RuntimeError("paged attention requires block_tables")

    if metadata.is_decode:
        if metadata.context_lens is None:
            raise RuntimeError("decode metadata requires context_lens")
        plan = None
        if metadata.context_lens.is_cuda:
            plan = metadata.decode_plan(key_cache.shape[2], key_cache.shape[1])
        return hip_paged_decode(
            query,
            key_cache,
            value_cache,
            metadata.block_tables,
            metadata.context_lens,
            scale=scale,
            plan=plan,
        )

    if metadata.cu_seqlens_q is None or metadata.cu_seqlens_k is None:
        raise RuntimeError("prefill metadata requires cu_seqlens_q and cu_seqlens_k")
    max_q = metadata.max_seqlen_q
    if max_q <= 0:
        max_q = max(metadata.q_lens_cpu, default=0)
    return hip_paged_prefill(
        query,
        key_cache,
        value_cache,
        metadata.cu_seqlens_q,
        metadata.cu_seqlens_k,
        metadata.block_tables,
        max_seqlen_q=max_q,
        scale=scale,
        plan=metadata.prefill_plan(query, key_cache),
    )


def varlen_attention(query, keys, values, metadata: AttentionMetadata, *, scale=None):
    """Causal varlen attention over contiguous K/V (no-prefix prefill).

    Serves the path the reference sends to FlashAttention varlen or a
    per-request SDPA loop (microinfer/layer/cached_attention.py:17-55, :87-101).
    """
    if query.shape[0] == 0:
        return torch.empty_like(query)
    if not query.is_cuda:
        raise RuntimeError(
            f"varlen attention runs on the HIP device only; got a {query.device} query"
        )
    cu_q = metadata.cu_seqlens_q
    cu_k = metadata.cu_seqlens_k if metadata.cu_seqlens_k is not None else cu_q
    if cu_q is None:
        raise RuntimeError("prefill metadata requires cu_seqlens_q")
    max_q = metadata.max_seqlen_q
    if max_q <= 0:
        max_q = max(metadata.q_lens_cpu, default=0)
    return hip_paged_prefill(
        query, keys, values, cu_q, cu_k, None, max_seqlen_q=max_q, scale=scale,
        plan=metadata.prefill_plan(query, keys, paged=False),
    )

"""The reference's paged-attention module, served by the gfx950 HIP kernels.

Same module name and exported names as microinfer/layer/triton_paged_attention.py,
so that code written against it -- the reference's own tests
(tests/layers/test_triton_paged_attention.py:3-8), its bench's backend labels
(bench/engines/microinfer.py:104-139) -- runs unchanged after its import
path is pointed here:

* ``triton_paged_decode`` (:352-457) and ``triton_paged_prefill``
  (:260-339): same positional and keyword arguments, the same ValueError
  preconditions in the same order, the same output (shape, dtype, a new
  tensor from ``torch.empty_like``-style allocation);
* ``HAS_TRITON`` (:26-34): True when the backend these two functions call
  is usable -- here, when ``libmi_attn.so`` loads. Without it both raise
  RuntimeError, as the reference does without Triton;
* ``DEFAULT_SPLIT_K``, ``MIN_PROGRAMS`` and ``_select_split_k`` (:342-349):
  the reference's host-side split choice, kept for callers that read it.

Differences, by design: ``split_k=None`` lets the device plan the context
partitions from ``context_lens`` (the reference picks 4 or 1 on the host);
an explicit ``split_k`` caps the partitions per sequence. The result does
not depend on the partitioning beyond float rounding (tested at 1e-5 in
fp32), and the launch shape depends only on the batch size, so a captured
hipGraph stays valid as contexts grow. Decode accepts fp32, fp16 and bf16 as
the reference does; prefill keeps the reference's FP16/BF16-only contract
here (``hip_paged_prefill`` itself also serves fp32 and contiguous K/V).
"""

from __future__ import annotations

import torch

from microinfer_amd import _lib
from microinfer_amd.layer.hip_paged_attention import hip_paged_decode, hip_paged_prefill


def _backend_loads() -> bool:
    try:
        _lib.load()
    except (OSError, RuntimeError):
        return False
    return True


# Named after the reference's capability flag (its bench labels the decode
# backend "triton" when this is set); the backend here is HIP.
HAS_TRITON = _backend_loads()
BACKEND = "hip-gfx950"

DEFAULT_SPLIT_K = 4
# Below this many (request, head) programs the reference's decode grid cannot
# fill the GPU, so it splits each head's scan.
MIN_PROGRAMS = 64


def _select_split_k(num_requests: int, num_q_heads: int) -> int:
    """The reference's host-side split choice (triton_paged_attention.py:348-349)."""
    return DEFAULT_SPLIT_K if num_requests * num_q_heads < MIN_PROGRAMS else 1


def _require_backend() -> None:
    if not HAS_TRITON:
        raise RuntimeError("the HIP paged-attention library (libmi_attn.so) is not available")


def triton_paged_decode(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    *,
    scale: float | None = None,
    split_k: int | None = None,
) -> torch.Tensor:
    """Decode one query per request over the paged KV cache (any power-of-two
    block size and head_dim; fp32, fp16 or bf16)."""
    _require_backend()
    if query.ndim != 3:
        raise ValueError("query must have shape [requests, Hq, D]")
    num_requests, num_q_heads, head_dim = query.shape
    _num_blocks, block_size, num_kv_heads, kv_dim = key_cache.shape
    if num_requests == 0:
        return torch.empty_like(query)
    if query.device != key_cache.device or query.dtype != key_cache.dtype:
        raise ValueError("query and cache must share device/dtype")
    if not query.is_cuda:
        raise ValueError("paged decode requires a GPU device")
    if query.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("unsupported query dtype")
    if kv_dim != head_dim:
        raise ValueError("query and cache head dimensions differ")
    if num_q_heads % num_kv_heads:
        raise ValueError("Hq must be divisible by Hkv")
    if block_size <= 0 or block_size & (block_size - 1):
        raise ValueError("paged decode requires a power-of-two block size")
    if head_dim <= 0 or head_dim & (head_dim - 1):
        raise ValueError("paged decode requires a power-of-two head_dim")
    if split_k is not None and (type(split_k) is not int or split_k <= 0
                                or split_k & (split_k - 1)):
        raise ValueError("split_k must be a positive power of two")
    if block_tables.shape[0] != num_requests:
        raise ValueError("block_tables must have one row per request")
    if context_lens.numel() != num_requests:
        raise ValueError("context_lens must have one entry per request")
    return hip_paged_decode(query, key_cache, value_cache, block_tables, context_lens,
                            scale=scale, split_k=split_k)


def triton_paged_prefill(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    block_tables: torch.Tensor,
    *,
    max_seqlen_q: int,
    scale: float | None = None,
) -> torch.Tensor:
    """Causal prefill straight from the paged cache (no gather copy),
    bottom-right aligned: row i of request r sees keys up to
    ``(c_r - q_r) + i``."""
    _require_backend()
    if query.ndim != 3:
        raise ValueError("query must have shape [tokens, Hq, D]")
    num_tokens, num_q_heads, head_dim = query.shape
    _num_blocks, block_size, num_kv_heads, kv_dim = key_cache.shape
    num_requests = block_tables.shape[0]
    if num_tokens == 0 or num_requests == 0:
        return torch.empty_like(query)
    if query.device != key_cache.device or query.dtype != key_cache.dtype:
        raise ValueError("query and cache must share device/dtype")
    if query.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("paged prefill requires FP16/BF16")
    if kv_dim != head_dim or head_dim % 16:
        raise ValueError("head dimension must match and be a multiple of 16")
    if num_q_heads % num_kv_heads:
        raise ValueError("Hq must be divisible by Hkv")
    if block_size <= 0 or block_size & (block_size - 1):
        raise ValueError("paged prefill requires a power-of-two block size")
    if cu_seqlens_q.numel() != num_requests + 1:
        raise ValueError("cu_seqlens_q must have num_requests + 1 entries")
    if cu_seqlens_k.numel() != num_requests + 1:
        raise ValueError("cu_seqlens_k must have num_requests + 1 entries")
    if max_seqlen_q <= 0:
        raise ValueError("max_seqlen_q must be positive")
    return hip_paged_prefill(query, key_cache, value_cache, cu_seqlens_q, cu_seqlens_k,
                             block_tables, max_seqlen_q=max_seqlen_q, scale=scale)

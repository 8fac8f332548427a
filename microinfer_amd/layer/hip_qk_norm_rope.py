"""Fused Q/K RMSNorm + RoPE + KV append through the HIP library.

One launch per layer and step for what ``Attention.forward`` does between the
fused QKV projection and the attention call
(microinfer/layer/transformer.py:186-233: ``q_norm``/``k_norm``
(norm.py:26-35), ``rotary.apply`` on Q and K (rope.py:6-20, :74-85)) plus the
append that ``CachedAttention.forward`` performs first
(microinfer/layer/cached_attention.py:76-85, worker/kv_cache.py:52-79).
Contract violations raise ValueError before anything is launched; a CPU
tensor raises RuntimeError (there is no CPU fallback).
"""

from __future__ import annotations

import torch

from microinfer_amd import _lib

_FLOAT_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def rope_tables(max_len: int, dim: int, base: float, *, device) -> tuple[torch.Tensor, torch.Tensor]:
    """float32 cos/sin tables ``[max_len, dim / 2]`` as ``RotaryCache.ensure``
    builds them (microinfer/layer/rope.py:45-55): ``inv = base ** (-arange(0,
    dim, 2) / dim)``, ``angles = outer(arange(max_len), inv)``."""
    if max_len <= 0 or dim <= 0 or dim % 2 or base <= 0:
        raise ValueError("invalid RoPE cache dimensions/base")
    inv = base ** (-torch.arange(0, dim, 2, device=device, dtype=torch.float32) / dim)
    angles = torch.outer(torch.arange(max_len, device=device, dtype=torch.float32), inv)
    return angles.cos(), angles.sin()


def qk_norm_rope_append(
    qkv: torch.Tensor,
    *,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    eps: float,
    cos_table: torch.Tensor,
    sin_table: torch.Tensor,
    positions: torch.Tensor,
    num_q_heads: int,
    num_kv_heads: int,
    head_dim: int,
    interleaved: bool = False,
    slot_mapping: torch.Tensor | None = None,
    key_cache: torch.Tensor | None = None,
    value_cache: torch.Tensor | None = None,
    return_k: bool = False,
):
    """Normalise and rotate Q and K of ``qkv [T, (Hq + 2 Hkv) * D]``.

    Returns ``q [T, Hq, D]`` (and ``k [T, Hkv, D]`` when ``return_k``). With
    ``slot_mapping`` (int32/int64 ``[T]``, -1 skipped) the rotated K rows and
    the projected V rows are written into ``key_cache`` / ``value_cache``
    (``[N, B, Hkv, D]``). ``cos_table`` / ``sin_table`` are the float32
    ``[max_len, D / 2]`` tables of ``RotaryCache.tables`` (rope.py:57-60).
    """
    _lib.require_device(qkv, q_weight, k_weight, cos_table, sin_table, positions,
                        slot_mapping, key_cache, value_cache, what="QK norm + RoPE")
    if qkv.dtype not in _FLOAT_DTYPES:
        raise ValueError("qkv must be float16, bfloat16 or float32")
    if num_q_heads <= 0 or num_kv_heads <= 0 or num_q_heads % num_kv_heads:
        raise ValueError("invalid GQA head ratio")
    lo = 2 * 16 // qkv.element_size()
    if head_dim < lo or head_dim > 256 or head_dim & (head_dim - 1):
        raise ValueError(f"head_dim must be a power of two in [{lo}, 256]")
    width = (num_q_heads + 2 * num_kv_heads) * head_dim
    if qkv.ndim != 2 or qkv.shape[1] < width or qkv.stride(1) != 1:
        raise ValueError("qkv must be [tokens, (Hq + 2 Hkv) * D] with contiguous rows")
    vec = 16 // qkv.element_size()
    if qkv.data_ptr() % 16 or (qkv.shape[0] > 1 and qkv.stride(0) % vec):
        qkv = qkv[:, :width].contiguous()  # rows move as aligned 16-byte vectors
    for name, w in (("q_weight", q_weight), ("k_weight", k_weight)):
        if w.shape != (head_dim,) or w.dtype != qkv.dtype:
            raise ValueError(f"{name} must be [head_dim] in the dtype of qkv")
    half = head_dim // 2
    for name, table in (("cos_table", cos_table), ("sin_table", sin_table)):
        if table.dtype != torch.float32 or table.ndim != 2 or table.shape[1] != half:
            raise ValueError(f"{name} must be float32 [max_len, head_dim / 2]")
    if cos_table.shape != sin_table.shape:
        raise ValueError("cos/sin tables differ in shape")
    tokens = qkv.shape[0]
    if positions.dtype not in (torch.int32, torch.int64) or positions.numel() != tokens:
        raise ValueError("positions must be int32/int64 with one entry per token")
    if slot_mapping is not None:
        if key_cache is None or value_cache is None:
            raise ValueError("an append needs both caches")
        if slot_mapping.numel() != tokens:
            raise ValueError("one slot per token is required")
        if key_cache.ndim != 4 or key_cache.shape != value_cache.shape:
            raise ValueError("K/V caches must have matching [blocks, B, Hkv, D] shapes")
        if key_cache.stride() != value_cache.stride() or key_cache.stride(-1) != 1:
            raise ValueError("K/V caches must share one layout with contiguous head_dim")
        if key_cache.shape[2:] != (num_kv_heads, head_dim) or key_cache.dtype != qkv.dtype:
            raise ValueError("caches must match the KV heads, head_dim and dtype")
        slot_mapping = slot_mapping.to(torch.int32).contiguous()
    q = torch.empty((tokens, num_q_heads, head_dim), dtype=qkv.dtype, device=qkv.device)
    k = (torch.empty((tokens, num_kv_heads, head_dim), dtype=qkv.dtype, device=qkv.device)
         if return_k else None)
    if tokens == 0:
        return (q, k) if return_k else q
    cos_table, sin_table = cos_table.contiguous(), sin_table.contiguous()
    if cos_table.data_ptr() % 16 or sin_table.data_ptr() % 16:  # angles load as float4
        cos_table, sin_table = cos_table.clone(), sin_table.clone()
    positions = positions.contiguous()
    q_weight, k_weight = q_weight.contiguous(), k_weight.contiguous()
    appending = slot_mapping is not None
    lib = _lib.load()
    status = lib.mi_qk_norm_rope_append(
        qkv.data_ptr(), qkv.stride(0), q_weight.data_ptr(), k_weight.data_ptr(), float(eps),
        cos_table.data_ptr(), sin_table.data_ptr(), cos_table.shape[0],
        positions.data_ptr(), int(positions.dtype == torch.int64),
        slot_mapping.data_ptr() if appending else None,
        q.data_ptr(), q.stride(0), q.stride(1),
        k.data_ptr() if k is not None else None,
        k.stride(0) if k is not None else 0, k.stride(1) if k is not None else 0,
        key_cache.data_ptr() if appending else None,
        value_cache.data_ptr() if appending else None,
        key_cache.stride(0) if appending else 0, key_cache.stride(1) if appending else 0,
        key_cache.stride(2) if appending else 0,
        tokens, num_q_heads, num_kv_heads, head_dim, int(bool(interleaved)),
        key_cache.shape[1] if appending else 0, key_cache.shape[0] if appending else 0,
        _lib.dtype_code(qkv.dtype), _lib.stream_handle(qkv.device),
    )
    _lib.check(status, "mi_qk_norm_rope_append")
    return (q, k) if return_k else q

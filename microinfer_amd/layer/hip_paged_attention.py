"""HIP paged attention ops for gfx950, called through libmi_attn.so.

Drop-ins for the reference's Triton entry points
(microinfer/layer/triton_paged_attention.py):

* ``hip_paged_decode``  <- ``triton_paged_decode``  (:352-457)
* ``hip_paged_prefill`` <- ``triton_paged_prefill`` (:260-339)

Same positional/keyword arguments, same ValueError checks (:280-302,
:370-399), same output dtype and shape. Differences by design:

* One launch handles all G = Hq/Hkv query heads of a KV head, so K/V is read
  from HBM once per step (the reference reads it G times).
* ``split_k=None`` plans context partitions on the device from
  ``context_lens`` (the reference picks 4 or 1 on the host from R*Hq); an int
  forces at most that many partitions per sequence. The launch shape depends
  only on the batch size, so hipGraph capture stays valid as contexts grow.
* Prefill also accepts float32 (vector kernel) and contiguous varlen K/V
  (``block_tables=None``), which serves the no-prefix prefill.

Workspace comes from torch's caching allocator (the graph pool under
capture); the library never allocates.
"""

from __future__ import annotations

from dataclasses import dataclass

import math

import torch

from microinfer_amd import _lib

_FLOAT_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _is_pow2(value: int) -> bool:
    return value > 0 and value & (value - 1) == 0


def _inner_contiguous(tensor: torch.Tensor) -> torch.Tensor:
    return tensor if tensor.stride(-1) == 1 else tensor.contiguous()


def _index32(tensor: torch.Tensor) -> torch.Tensor:
    if tensor.dtype != torch.int32:
        tensor = tensor.to(torch.int32)
    return tensor.contiguous()


def _check_caches(key_cache: torch.Tensor, value_cache: torch.Tensor):
    if key_cache.ndim != 4 or value_cache.shape != key_cache.shape:
        raise ValueError("key/value caches must have matching [blocks, B, Hkv, D] shapes")
    if value_cache.dtype != key_cache.dtype or value_cache.device != key_cache.device:
        raise ValueError("key/value caches must share dtype and device")
    key_cache = _inner_contiguous(key_cache)
    value_cache = _inner_contiguous(value_cache)
    if key_cache.stride() != value_cache.stride():
        # The kernels address K and V with one set of strides.
        key_cache = key_cache.contiguous()
        value_cache = value_cache.contiguous()
    return key_cache, value_cache


# Split-merge arrival counters: one zero-filled int32 array per (device,
# stream). Every decode launch leaves its counters zero again, so the array is
# reused by all later calls on that stream (including graph replays). A grown
# array replaces the old one, which stays alive because captured graphs may
# still point at it.
_counters: dict[tuple[int, int], torch.Tensor] = {}
_retired_counters: list[torch.Tensor] = []


_PLAN_READY = 1  # MI_PREFILL_PLAN_READY
_cus: dict[int, int] = {}


def _device_cus(device: torch.device) -> int:
    index = device.index if device.index is not None else torch.cuda.current_device()
    if index not in _cus:
        _cus[index] = torch.cuda.get_device_properties(index).multi_processor_count
    return _cus[index]


def _decode_counters(device: torch.device, stream: int, needed: int) -> torch.Tensor:
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    counters = _counters.get(key)
    if counters is None or counters.numel() < needed:
        if counters is not None:
            _retired_counters.append(counters)
        counters = torch.zeros(max(needed, 4096), dtype=torch.int32, device=device)
        _counters[key] = counters
    return counters


def decode_workspace_bytes(num_seqs: int, num_q_heads: int, num_kv_heads: int,
                           head_dim: int, split_k: int | None) -> int:
    return int(
        _lib.load().mi_paged_decode_workspace_bytes(
            num_seqs, num_q_heads, num_kv_heads, head_dim, 0 if split_k is None else split_k
        )
    )


def decode_plan(context_lens: torch.Tensor, *, num_kv_heads: int, block_size: int,
                block_table_width: int, split_k: int | None = None) -> torch.Tensor:
    """Partition plan for one decode step (shared by every layer of the step).

    Computed on the device from ``context_lens`` (int32 ``[R]``), so it can be
    captured in a hipGraph; pass it to ``hip_paged_decode(..., plan=...)``.
    """
    _lib.require_device(context_lens, what="decode_plan")
    context_lens = _index32(context_lens)
    num_seqs = context_lens.numel()
    split = 0 if split_k is None else split_k
    lib = _lib.load()
    nbytes = int(lib.mi_decode_plan_bytes(num_seqs, num_kv_heads, split))
    plan = torch.empty(max(nbytes, 32), dtype=torch.uint8, device=context_lens.device)
    status = lib.mi_decode_plan(
        context_lens.data_ptr(), num_seqs, num_kv_heads, block_size, block_table_width, split,
        plan.data_ptr(), plan.numel(), _lib.stream_handle(context_lens.device),
    )
    _lib.check(status, "mi_decode_plan")
    return plan


def hip_paged_decode(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    *,
    scale: float | None = None,
    split_k: int | None = None,
    plan: torch.Tensor | None = None,
    new_keys: torch.Tensor | None = None,
    new_values: torch.Tensor | None = None,
) -> torch.Tensor:
    """Decode one query row per request over the paged cache.

    ``query [R, Hq, D]``, caches ``[N, B, Hkv, D]`` (any strides with D
    contiguous), ``block_tables [R, W]`` and ``context_lens [R]`` on the device.
    Returns ``[R, Hq, D]`` in the query dtype. ``plan`` is an optional
    ``decode_plan(...)`` result for this step (same lengths, table width,
    KV heads and split_k); without it the call computes its own.

    ``new_keys`` / ``new_values`` (``[R, Hkv, D]``) fuse the step's KV append
    into the launch: row r is stored at cache position ``context_lens[r] - 1``
    (the slot the runner assigns a decode token, microinfer/runner.py:167-174)
    before it is attended, as CachedAttention.forward's append-then-attend
    does (microinfer/layer/cached_attention.py:76-85). The caches are then
    written in place and must share strides.
    """
    if query.ndim != 3:
        raise ValueError("query must have shape [requests, Hq, D]")
    num_requests, num_q_heads, head_dim = query.shape
    if key_cache.ndim != 4:
        raise ValueError("key_cache must have shape [blocks, B, Hkv, D]")
    num_blocks, block_size, num_kv_heads, kv_dim = key_cache.shape
    if num_requests == 0:
        return torch.empty_like(query)
    if query.device != key_cache.device or query.dtype != key_cache.dtype:
        raise ValueError("query and cache must share device/dtype")
    if not query.is_cuda:
        raise ValueError("HIP paged decode requires a GPU device")
    if query.dtype not in _FLOAT_DTYPES:
        raise ValueError("unsupported query dtype")
    if kv_dim != head_dim:
        raise ValueError("query and cache head dimensions differ")
    if num_q_heads % num_kv_heads:
        raise ValueError("Hq must be divisible by Hkv")
    if not _is_pow2(block_size):
        raise ValueError("paged kernels require a power-of-two block size")
    if not _is_pow2(head_dim):
        raise ValueError("paged kernels require a power-of-two head_dim")
    if split_k is not None and (type(split_k) is not int or not _is_pow2(split_k)):
        raise ValueError("split_k must be a positive power of two")
    if block_tables.ndim != 2 or block_tables.shape[0] != num_requests:
        raise ValueError("block_tables must have one row per request")
    if context_lens.numel() != num_requests:
        raise ValueError("context_lens must have one entry per request")
    _lib.require_device(block_tables, context_lens, what="hip_paged_decode")

    append = new_keys is not None or new_values is not None
    if append:
        if new_keys is None or new_values is None:
            raise ValueError("new_keys and new_values must be given together")
        for name, rows in (("new_keys", new_keys), ("new_values", new_values)):
            if rows.shape != (num_requests, num_kv_heads, head_dim):
                raise ValueError(f"{name} must have shape [requests, Hkv, D]")
            if rows.dtype != query.dtype or rows.device != query.device:
                raise ValueError(f"{name} must share the query's dtype and device")
        if (key_cache.stride(-1) != 1 or value_cache.stride(-1) != 1
                or key_cache.stride() != value_cache.stride()):
            raise ValueError("an appending decode writes the caches in place: they need "
                             "equal strides with a contiguous head_dim")
        new_keys = _inner_contiguous(new_keys)
        new_values = _inner_contiguous(new_values)
    key_cache, value_cache = _check_caches(key_cache, value_cache)
    query = _inner_contiguous(query)
    block_tables = _index32(block_tables)
    context_lens = _index32(context_lens)
    output = torch.empty(query.shape, dtype=query.dtype, device=query.device)
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)

    lib = _lib.load()
    split = 0 if split_k is None else split_k
    ws_bytes = int(
        lib.mi_paged_decode_workspace_bytes(
            num_requests, num_q_heads, num_kv_heads, head_dim, split
        )
    )
    stream = _lib.stream_handle(query.device)
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=query.device)
    counters = _decode_counters(query.device, stream, num_requests * num_kv_heads)
    if plan is not None:
        _lib.require_device(plan, what="hip_paged_decode")
        if plan.dtype != torch.uint8 or not plan.is_contiguous():
            raise ValueError("plan must come from decode_plan()")
    args = (
        query.data_ptr(), query.stride(0), query.stride(1),
        key_cache.data_ptr(), value_cache.data_ptr(),
        key_cache.stride(0), key_cache.stride(1), key_cache.stride(2),
        block_tables.data_ptr(), block_tables.stride(0), block_tables.shape[1],
        context_lens.data_ptr(),
        output.data_ptr(), output.stride(0), output.stride(1),
        workspace.data_ptr(), ws_bytes, counters.data_ptr(),
        None if plan is None else plan.data_ptr(), 0 if plan is None else plan.numel(),
        num_requests, num_q_heads, num_kv_heads, head_dim, block_size, num_blocks,
        split, float(scale), _lib.dtype_code(query.dtype), stream,
    )
    if append:
        status = lib.mi_paged_decode_append(
            new_keys.data_ptr(), new_keys.stride(0), new_keys.stride(1),
            new_values.data_ptr(), new_values.stride(0), new_values.stride(1), *args)
        _lib.check(status, "mi_paged_decode_append")
    else:
        status = lib.mi_paged_decode(*args)
        _lib.check(status, "mi_paged_decode")
    return output


@dataclass(frozen=True)
class PrefillPlan:
    """Launch plan of planned prefill calls (``prefill_plan``): the workspace
    it was written into and the call sizes it was made for."""

    workspace: torch.Tensor
    key: tuple


def _prefill_key(num_tokens, num_requests, num_q_heads, num_kv_heads, head_dim, dtype, paged,
                 block_size, block_table_width, num_blocks) -> tuple:
    return (num_tokens, num_requests, num_q_heads, num_kv_heads, head_dim, dtype, bool(paged),
            block_size if paged else 0, block_table_width if paged else 0,
            0 if paged else num_blocks)


def prefill_plan(cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor, *, num_tokens: int,
                 num_q_heads: int, num_kv_heads: int, head_dim: int, dtype: torch.dtype,
                 block_size: int = 0, block_table_width: int = 0,
                 num_kv_rows: int = 0, paged: bool = True) -> PrefillPlan | None:
    """Launch plan for the prefill calls of one step (shared by every layer).

    Computed on the device from the cu_seqlens (so a hipGraph can hold it);
    pass it to ``hip_paged_prefill(..., plan=...)`` for calls with these sizes
    (paged: block tables of width ``block_table_width``; contiguous K/V:
    ``num_kv_rows`` rows). None when these sizes run unplanned.
    """
    _lib.require_device(cu_seqlens_q, cu_seqlens_k, what="prefill_plan")
    cu_seqlens_q = _index32(cu_seqlens_q)
    cu_seqlens_k = _index32(cu_seqlens_k)
    num_requests = cu_seqlens_q.numel() - 1
    lib = _lib.load()
    code = _lib.dtype_code(dtype)
    nbytes = lib.mi_paged_prefill_workspace_bytes(num_tokens, num_requests, num_q_heads,
                                                  num_kv_heads, head_dim, code)
    if nbytes <= 0:
        return None
    workspace = torch.empty(nbytes, dtype=torch.uint8, device=cu_seqlens_q.device)
    status = lib.mi_paged_prefill_plan(
        cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(), num_tokens, num_requests, num_q_heads,
        num_kv_heads, head_dim, int(paged), block_size, block_table_width, num_kv_rows, code,
        workspace.data_ptr(), nbytes, _lib.stream_handle(cu_seqlens_q.device),
    )
    _lib.check(status, "mi_paged_prefill_plan")
    key = _prefill_key(num_tokens, num_requests, num_q_heads, num_kv_heads, head_dim, code,
                       paged, block_size, block_table_width, num_kv_rows)
    return PrefillPlan(workspace, key)


def hip_paged_prefill(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    block_tables: torch.Tensor | None,
    *,
    max_seqlen_q: int,
    scale: float | None = None,
    planned: bool = True,
    plan: PrefillPlan | None = None,
) -> torch.Tensor:
    """Causal varlen attention straight from the paged cache (bottom-right mask).

    ``query [T, Hq, D]``; request r owns query rows ``cu_seqlens_q[r]..`` and
    context ``cu_seqlens_k[r+1] - cu_seqlens_k[r]`` (it includes the new rows,
    which the caller appended first). With ``block_tables=None`` the "caches"
    are contiguous ``[sum c, Hkv, D]`` K/V and request r's keys start at row
    ``cu_seqlens_k[r]``.

    ``planned`` (default) runs the MFMA kernel behind a launch plan
    (``mi_paged_prefill_planned``: long items split along their keys, largest
    first) when the call has fewer (query block, KV head) items than two per
    CU, else unplanned; False always runs ``mi_paged_prefill``, one
    workgroup per (query block, KV head) and no workspace. Both agree to
    float rounding. ``plan``: a ``prefill_plan(...)`` result for this call's
    cu_seqlens and sizes, which skips the plan kernel (one plan per step
    serves every layer) and is always used.
    """
    if query.ndim != 3:
        raise ValueError("query must have shape [tokens, Hq, D]")
    num_tokens, num_q_heads, head_dim = query.shape
    paged = block_tables is not None
    if paged:
        if key_cache.ndim != 4:
            raise ValueError("key_cache must have shape [blocks, B, Hkv, D]")
        num_blocks, block_size, num_kv_heads, kv_dim = key_cache.shape
        num_requests = block_tables.shape[0]
    else:
        if key_cache.ndim != 3 or value_cache.shape != key_cache.shape:
            raise ValueError("contiguous K/V must have shape [rows, Hkv, D]")
        num_blocks, num_kv_heads, kv_dim = key_cache.shape
        block_size = 1
        num_requests = cu_seqlens_q.numel() - 1
    if num_tokens == 0 or num_requests == 0:
        return torch.empty_like(query)
    if query.device != key_cache.device or query.dtype != key_cache.dtype:
        raise ValueError("query and cache must share device/dtype")
    if not query.is_cuda:
        raise ValueError("HIP paged prefill requires a GPU device")
    if query.dtype not in _FLOAT_DTYPES:
        raise ValueError("unsupported query dtype")
    if kv_dim != head_dim or not _is_pow2(head_dim):
        raise ValueError("head dimension must match and be a power of two")
    if num_q_heads % num_kv_heads:
        raise ValueError("Hq must be divisible by Hkv")
    if not _is_pow2(block_size):
        raise ValueError("paged kernels require a power-of-two block size")
    if cu_seqlens_q.numel() != num_requests + 1:
        raise ValueError("cu_seqlens_q must have num_requests + 1 entries")
    if cu_seqlens_k.numel() != num_requests + 1:
        raise ValueError("cu_seqlens_k must have num_requests + 1 entries")
    if max_seqlen_q <= 0:
        raise ValueError("max_seqlen_q must be positive")
    _lib.require_device(cu_seqlens_q, cu_seqlens_k, block_tables, what="hip_paged_prefill")

    query = _inner_contiguous(query)
    if paged:
        key_cache, value_cache = _check_caches(key_cache, value_cache)
        block_tables = _index32(block_tables)
        c_bs, c_ts, c_hs = key_cache.stride(0), key_cache.stride(1), key_cache.stride(2)
        t_ptr, t_stride, t_width = block_tables.data_ptr(), block_tables.stride(0), block_tables.shape[1]
    else:
        key_cache = _inner_contiguous(key_cache)
        value_cache = _inner_contiguous(value_cache)
        if key_cache.stride() != value_cache.stride():
            key_cache, value_cache = key_cache.contiguous(), value_cache.contiguous()
        c_bs, c_ts, c_hs = 0, key_cache.stride(0), key_cache.stride(1)
        t_ptr, t_stride, t_width = None, 0, 0
        # The kernel never reads past this many K/V rows.
        num_blocks = max(num_blocks, 1)
    cu_seqlens_q = _index32(cu_seqlens_q)
    cu_seqlens_k = _index32(cu_seqlens_k)
    output = torch.empty(query.shape, dtype=query.dtype, device=query.device)
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)

    lib = _lib.load()
    dtype = _lib.dtype_code(query.dtype)
    flags = 0
    if plan is not None:
        if not planned:
            raise ValueError("a plan needs planned=True")
        key = _prefill_key(num_tokens, num_requests, num_q_heads, num_kv_heads, head_dim, dtype,
                           paged, block_size, t_width, num_blocks)
        if not isinstance(plan, PrefillPlan) or plan.key != key:
            raise ValueError("plan must come from prefill_plan() with this call's sizes")
        _lib.require_device(plan.workspace, what="hip_paged_prefill")
        workspace, ws_bytes, flags = plan.workspace, plan.workspace.numel(), _PLAN_READY
    else:
        # A call that plans for itself pays the plan kernel (≈ 7 µs): worth
        # it only where the launch is short of items to keep two workgroups
        # on every CU (there the plan splits long items: one 8192-token
        # request 207 → 64 µs); with more items the unplanned order is
        # within a few per cent. A plan shared by a step's layers
        # (``plan=``) always pays off.
        if planned:
            rows_per_block = 128 * num_kv_heads // num_q_heads if num_q_heads else 128
            items = (num_tokens // max(rows_per_block, 1) + num_requests) * num_kv_heads
            planned = items < 2 * _device_cus(query.device)
        # The launch plan's workspace (split partials, the plan, its
        # counters): from the caching allocator, so a captured graph owns it.
        ws_bytes = (lib.mi_paged_prefill_workspace_bytes(num_tokens, num_requests, num_q_heads,
                                                         num_kv_heads, head_dim, dtype)
                    if planned else 0)
        workspace = (torch.empty(ws_bytes, dtype=torch.uint8, device=query.device)
                     if ws_bytes > 0 else None)
    status = lib.mi_paged_prefill_planned(
        query.data_ptr(), query.stride(0), query.stride(1),
        key_cache.data_ptr(), value_cache.data_ptr(), c_bs, c_ts, c_hs,
        cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(), t_ptr, t_stride, t_width,
        output.data_ptr(), output.stride(0), output.stride(1),
        num_tokens, num_requests, int(max_seqlen_q), num_q_heads, num_kv_heads, head_dim,
        block_size, num_blocks, float(scale), dtype,
        workspace.data_ptr() if workspace is not None else None, ws_bytes, flags,
        _lib.stream_handle(query.device),
    )
    _lib.check(status, "mi_paged_prefill_planned")
    return output


def hip_gather_kv(key_cache, value_cache, block_tables, cu_seqlens_k, total_rows: int):
    """One-launch gather of each request's valid rows into contiguous K/V."""
    _lib.require_device(key_cache, value_cache, block_tables, cu_seqlens_k, what="gather_kv")
    key_cache, value_cache = _check_caches(key_cache, value_cache)
    num_blocks, block_size, num_kv_heads, head_dim = key_cache.shape
    if not _is_pow2(block_size):
        raise ValueError("paged kernels require a power-of-two block size")
    block_tables = _index32(block_tables)
    cu_seqlens_k = _index32(cu_seqlens_k)
    shape = (total_rows, num_kv_heads, head_dim)
    keys = torch.empty(shape, dtype=key_cache.dtype, device=key_cache.device)
    values = torch.empty_like(keys)
    if total_rows == 0:
        return keys, values
    status = _lib.load().mi_gather_kv(
        key_cache.data_ptr(), value_cache.data_ptr(),
        key_cache.stride(0), key_cache.stride(1), key_cache.stride(2),
        block_tables.data_ptr(), block_tables.stride(0), block_tables.shape[1],
        cu_seqlens_k.data_ptr(), block_tables.shape[0], total_rows,
        keys.data_ptr(), values.data_ptr(), num_kv_heads, head_dim, block_size, num_blocks,
        _lib.dtype_code(key_cache.dtype), _lib.stream_handle(key_cache.device),
    )
    _lib.check(status, "mi_gather_kv")
    return keys, values

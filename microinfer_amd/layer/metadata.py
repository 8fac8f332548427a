"""Per-step attention metadata.

Mirrors ``AttentionMetadata`` (microinfer/layer/metadata.py:17-116): the same
fields, ``build`` factory, lazily cached CPU tuples and ``slot_indices``. The
HIP append reads ``slot_mapping`` (int32) directly, so ``slot_indices`` is kept
only for callers of ``LayerKVCache.write_fast``.

Device index tensors are int32 (block tables ``[R, W]`` padded with -1,
context lengths ``[R]``, cu_seqlens ``[R + 1]``, slots ``[T]``), which is what
the kernels read without conversion.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch


@dataclass
class AttentionMetadata:
    is_prefill: bool
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None
    direct_prefill: bool = False
    validate_cache_write: bool = True
    _cu_q_cpu: tuple[int, ...] | None = field(default=None, repr=False)
    _context_lens_cpu: tuple[int, ...] | None = field(default=None, repr=False)
    _q_lens_cpu: tuple[int, ...] | None = field(default=None, repr=False)
    _slot_mapping_long: torch.Tensor | None = field(default=None, repr=False)
    _slot_block_size: int | None = field(default=None, repr=False)
    _slot_blocks: torch.Tensor | None = field(default=None, repr=False)
    _slot_offsets: torch.Tensor | None = field(default=None, repr=False)
    _decode_plans: dict = field(default_factory=dict, repr=False)
    _prefill_plans: dict = field(default_factory=dict, repr=False)

    @classmethod
    def build(
        cls,
        *,
        is_prefill: bool,
        cu_seqlens_q=None,
        cu_seqlens_k=None,
        max_seqlen_q: int = 0,
        max_seqlen_k: int = 0,
        slot_mapping=None,
        context_lens=None,
        block_tables=None,
        validate_cache_write: bool = True,
    ) -> "AttentionMetadata":
        """Same factory as metadata.py:36-61; no-prefix prefill has no table."""
        return cls(
            is_prefill=is_prefill,
            cu_seqlens_q=cu_seqlens_q,
            cu_seqlens_k=cu_seqlens_k,
            max_seqlen_q=max_seqlen_q,
            max_seqlen_k=max_seqlen_k,
            slot_mapping=slot_mapping,
            context_lens=context_lens,
            block_tables=block_tables,
            direct_prefill=is_prefill and block_tables is None,
            validate_cache_write=validate_cache_write,
        )

    @property
    def is_decode(self) -> bool:
        return not self.is_prefill

    @property
    def slot_mapping_long(self) -> torch.Tensor:
        if self.slot_mapping is None:
            raise ValueError("metadata has no slot_mapping")
        if self._slot_mapping_long is None:
            self._slot_mapping_long = self.slot_mapping.long()
        return self._slot_mapping_long

    def slot_indices(self, block_size: int) -> tuple[torch.Tensor, torch.Tensor]:
        """(block, offset) tensors with floor semantics, cached per block size."""
        if block_size <= 0:
            raise ValueError("block_size must be positive")
        if self._slot_block_size != block_size:
            slots = self.slot_mapping_long
            blocks = torch.div(slots, block_size, rounding_mode="floor")
            self._slot_blocks = blocks
            self._slot_offsets = slots - blocks * block_size
            self._slot_block_size = block_size
        return self._slot_blocks, self._slot_offsets

    def decode_plan(self, num_kv_heads: int, block_size: int) -> torch.Tensor:
        """Device partition plan for this decode step, built once and reused
        by every layer (like ``slot_indices``)."""
        if self.context_lens is None or self.block_tables is None:
            raise ValueError("decode plan needs context_lens and block_tables")
        from microinfer_amd.layer.hip_paged_attention import decode_plan

        key = (num_kv_heads, block_size, self.block_tables.shape[1])
        plan = self._decode_plans.get(key)
        if plan is None:
            plan = decode_plan(self.context_lens, num_kv_heads=num_kv_heads,
                               block_size=block_size, block_table_width=key[2])
            self._decode_plans[key] = plan
        return plan

    def prefill_plan(self, query: torch.Tensor, key_cache: torch.Tensor, *, paged: bool = True):
        """Device launch plan for this step's prefill calls, built once and
        reused by every layer (None where such calls run unplanned)."""
        if self.cu_seqlens_q is None or not self.cu_seqlens_q.is_cuda:
            return None
        from microinfer_amd.layer.hip_paged_attention import prefill_plan

        num_tokens, num_q_heads, head_dim = query.shape
        if paged:
            if self.block_tables is None:
                return None
            _, block_size, num_kv_heads, _ = key_cache.shape
            width, rows = self.block_tables.shape[1], 0
        else:
            block_size, width = 0, 0
            rows, num_kv_heads = max(key_cache.shape[0], 1), key_cache.shape[1]
        key = (num_tokens, num_q_heads, num_kv_heads, head_dim, query.dtype, paged, block_size,
               width, rows)
        if key not in self._prefill_plans:
            cu_k = self.cu_seqlens_k if self.cu_seqlens_k is not None else self.cu_seqlens_q
            self._prefill_plans[key] = prefill_plan(
                self.cu_seqlens_q, cu_k, num_tokens=num_tokens, num_q_heads=num_q_heads,
                num_kv_heads=num_kv_heads, head_dim=head_dim, dtype=query.dtype,
                block_size=block_size, block_table_width=width, num_kv_rows=rows, paged=paged)
        return self._prefill_plans[key]

    @property
    def cu_q_cpu(self) -> tuple[int, ...]:
        if self._cu_q_cpu is None:
            if self.cu_seqlens_q is not None:
                self._cu_q_cpu = tuple(int(x) for x in self.cu_seqlens_q.tolist())
            elif self.context_lens is not None:
                self._cu_q_cpu = tuple(range(self.context_lens.numel() + 1))
            else:
                self._cu_q_cpu = (0,)
        return self._cu_q_cpu

    @property
    def context_lens_cpu(self) -> tuple[int, ...]:
        if self._context_lens_cpu is None:
            if self.context_lens is not None:
                self._context_lens_cpu = tuple(int(x) for x in self.context_lens.tolist())
            elif self.cu_seqlens_k is not None:
                ends = [int(x) for x in self.cu_seqlens_k.tolist()]
                self._context_lens_cpu = tuple(b - a for a, b in zip(ends, ends[1:]))
            else:
                self._context_lens_cpu = ()
        return self._context_lens_cpu

    @property
    def q_lens_cpu(self) -> tuple[int, ...]:
        if self._q_lens_cpu is None:
            cu = self.cu_q_cpu
            self._q_lens_cpu = tuple(b - a for a, b in zip(cu, cu[1:]))
        return self._q_lens_cpu

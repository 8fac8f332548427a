"""Test helpers: tensor <-> numpy bridges and oracle-backed expectations."""

from __future__ import annotations

import numpy as np
import torch

from oracle import paged_attention_reference

DTYPES = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
TOLERANCE = {torch.float32: 2e-3, torch.float16: 2e-2, torch.bfloat16: 2e-2}


def as_f32(tensor: torch.Tensor) -> np.ndarray:
    """Exact float32 copy of a float tensor on the host."""
    return tensor.detach().to("cpu", torch.float32).numpy()


def bits(tensor: torch.Tensor) -> np.ndarray:
    """Raw bit patterns of a tensor (for bit-exact comparisons)."""
    t = tensor.detach().cpu().contiguous()
    view = {4: torch.int32, 2: torch.int16, 8: torch.int64}[t.element_size()]
    return t.view(view).numpy()


def rounded(array: np.ndarray, dtype: torch.dtype, device) -> torch.Tensor:
    """Host float32 array -> tensor of ``dtype`` on ``device`` (round once)."""
    return torch.from_numpy(np.ascontiguousarray(array, dtype=np.float32)).to(dtype).to(device)


def oracle_attention(query, key_cache, value_cache, block_tables, contexts, cu_q, scale):
    """Oracle output for device/host tensors (inputs widened exactly to f32)."""
    tables = block_tables.cpu().numpy() if torch.is_tensor(block_tables) else np.asarray(block_tables)
    contexts = [int(c) for c in (contexts.tolist() if torch.is_tensor(contexts) else contexts)]
    cu_q = [int(c) for c in (cu_q.tolist() if torch.is_tensor(cu_q) else cu_q)]
    return paged_attention_reference(
        as_f32(query), as_f32(key_cache), as_f32(value_cache), tables, contexts, cu_q,
        scale=scale,
    )


def max_abs(actual: torch.Tensor, expected: np.ndarray) -> float:
    diff = np.abs(as_f32(actual) - expected)
    return float(diff.max()) if diff.size else 0.0


def compact_oracle_inputs(key_cache, value_cache, block_tables, contexts):
    """Copy only the referenced blocks to the host, with remapped tables.

    Lets the oracle run against multi-GB pools: the result is identical
    because attention only reads the referenced blocks.
    """
    tables = block_tables.cpu().numpy()
    contexts = [int(c) for c in (contexts.tolist() if torch.is_tensor(contexts) else contexts)]
    bsz = key_cache.shape[1]
    used = sorted({int(b) for r, c in enumerate(contexts) for b in tables[r, : (c + bsz - 1) // bsz]})
    remap = {b: i for i, b in enumerate(used)}
    new_tables = np.full_like(tables, -1)
    for r, c in enumerate(contexts):
        for j in range((c + bsz - 1) // bsz):
            new_tables[r, j] = remap[int(tables[r, j])]
    index = torch.tensor(used, dtype=torch.long, device=key_cache.device)
    k = as_f32(key_cache.index_select(0, index))
    v = as_f32(value_cache.index_select(0, index))
    return k, v, new_tables, contexts


def oracle_decode(query, key_cache, value_cache, block_tables, context_lens, scale):
    k, v, tables, contexts = compact_oracle_inputs(key_cache, value_cache, block_tables, context_lens)
    cu = list(range(len(contexts) + 1))
    return paged_attention_reference(as_f32(query), k, v, tables, contexts, cu, scale=scale)


def oracle_prefill(query, key_cache, value_cache, block_tables, contexts, cu_q, scale):
    k, v, tables, contexts = compact_oracle_inputs(key_cache, value_cache, block_tables, contexts)
    cu_q = [int(c) for c in (cu_q.tolist() if torch.is_tensor(cu_q) else cu_q)]
    return paged_attention_reference(as_f32(query), k, v, tables, contexts, cu_q, scale=scale)


def checked_paged_attention(query, key_cache, value_cache, block_tables, context_lens,
                            cu_seqlens_q, *, scale=None):
    """Validated entry used by the restated reference tests.

    Same contract as the reference's test-only strict entry
    (tests/support/attention.py:13-142): shape/device/dtype checks, table
    coverage, then metadata for ``paged_attention_meta``.
    """
    from microinfer_amd.layer.metadata import AttentionMetadata
    from microinfer_amd.layer.paged_attention import paged_attention_meta

    if query.ndim != 3 or key_cache.ndim != 4 or key_cache.shape != value_cache.shape:
        raise ValueError("bad query/cache shapes")
    num_q_heads, head_dim = query.shape[1:]
    num_blocks, block_size, num_kv_heads, kv_dim = key_cache.shape
    if kv_dim != head_dim or num_q_heads % num_kv_heads:
        raise ValueError(f"Hq={num_q_heads} must be divisible by Hkv={num_kv_heads}")
    cu_q = [int(x) for x in cu_seqlens_q.tolist()]
    contexts = [int(x) for x in context_lens.tolist()]
    if cu_q[0] != 0 or cu_q[-1] != query.shape[0] or len(cu_q) != len(contexts) + 1:
        raise ValueError("bad cu_seqlens_q")
    q_lens = [b - a for a, b in zip(cu_q, cu_q[1:])]
    for i, (q_len, c) in enumerate(zip(q_lens, contexts)):
        if q_len < 0 or c < 0 or q_len > c:
            raise ValueError(f"request {i}: query_len={q_len} exceeds context_len={c}")
        need = (c + block_size - 1) // block_size
        if need > block_tables.shape[1]:
            raise ValueError("block table too short")
        for block in block_tables[i, :need].tolist():
            if not 0 <= int(block) < num_blocks:
                raise ValueError(f"invalid block id {block}")
    if query.shape[0] == 0:
        return torch.empty_like(query)
    is_decode = all(q == 1 for q in q_lens)
    cu_k = None
    if not is_decode:
        offsets = [0]
        for c in contexts:
            offsets.append(offsets[-1] + c)
        cu_k = torch.tensor(offsets, dtype=torch.int32, device=query.device)
    metadata = AttentionMetadata(
        is_prefill=not is_decode,
        cu_seqlens_q=cu_seqlens_q,
        cu_seqlens_k=cu_k,
        max_seqlen_q=max(q_lens),
        max_seqlen_k=max(contexts),
        context_lens=context_lens,
        block_tables=block_tables,
        validate_cache_write=False,
        _cu_q_cpu=tuple(cu_q),
        _context_lens_cpu=tuple(contexts),
        _q_lens_cpu=tuple(q_lens),
    )
    return paged_attention_meta(query, key_cache, value_cache, metadata, scale=scale)


class FakeSeq:
    """The attributes of ``Sequence`` (microinfer/engine/sequence.py:14-45)
    that the runner's metadata build reads, like the reference tests'
    ``sequence_cls`` fixture."""

    def __init__(self, token_ids):
        self.token_ids = list(token_ids)
        self.last_token = self.token_ids[-1]
        self.num_cached_tokens = 0
        self.num_scheduled_tokens = 0
        self.block_table = []

    def __len__(self):
        return len(self.token_ids)

    def __getitem__(self, key):
        return self.token_ids[key]

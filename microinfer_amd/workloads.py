"""Seeded synthetic paged-attention workloads and their algorithmic cost.

One generator serves the GPU bench, the parity tests and the CPU baseline, so
all three see identical inputs. Draw order (numpy PCG64, seed 0):

1. context lengths ``c_r ~ U{lo..hi}`` (inclusive);
2. ``perm = rng.permutation(pool_blocks)``; sequence r takes the next
   ``ceil(c_r / B)`` ids of ``perm`` (tables never overlap), padded with -1;
3. Q ``N(0,1) [R, Hq, D]``;
4. K pool then V pool ``N(0,1) [N, B, Hkv, D]`` (host draw, small pools only);
5. new-token K then V ``N(0,1) [R, Hkv, D]``;
6. ``slot_r = table[r][(c_r-1) // B] * B + (c_r-1) % B`` -- the append writes
   position ``c_r - 1`` and attention reads ``c_r`` tokens, as
   microinfer/runner.py:167-174 builds decode rows.

Values are drawn in float32 and rounded to the target dtype afterwards.
Pools too large to draw on the host (the 28-layer decode workload: 30 GB) are
filled on the device with ``torch.randn`` under a seeded device generator;
the host copy of any block that a CPU check needs is read back from the
device, so CPU and GPU still agree bit for bit.

Shapes (Qwen3 attention): 0.6B = 16 Q / 8 KV heads, 8B = 32 Q / 8 KV heads,
head_dim 128, block 16.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

QWEN3_06B = dict(num_q_heads=16, num_kv_heads=8, head_dim=128)
QWEN3_8B = dict(num_q_heads=32, num_kv_heads=8, head_dim=128)


@dataclass
class DecodeBatch:
    """Metadata and (optionally) host tensors of one decode step."""

    context_lens: np.ndarray  # int32 [R]
    block_tables: np.ndarray  # int32 [R, W], -1 padded
    slots: np.ndarray  # int32 [R]
    block_size: int
    pool_blocks: int
    query: np.ndarray | None = None  # float32 [R, Hq, D]
    key_pool: np.ndarray | None = None  # float32 [N, B, Hkv, D]
    value_pool: np.ndarray | None = None
    new_keys: np.ndarray | None = None  # float32 [R, Hkv, D]
    new_values: np.ndarray | None = None
    meta: dict = field(default_factory=dict)


def draw_tables(rng, contexts, pool_blocks: int, block_size: int, width: int | None = None):
    """Non-overlapping block tables from one permutation of the pool."""
    need = [(int(c) + block_size - 1) // block_size for c in contexts]
    if sum(need) > pool_blocks:
        raise ValueError("pool too small for the requested contexts")
    perm = rng.permutation(pool_blocks)
    width = max(need, default=0) if width is None else width
    tables = np.full((len(contexts), max(width, 1)), -1, dtype=np.int32)
    cursor = 0
    for r, n in enumerate(need):
        tables[r, :n] = perm[cursor : cursor + n]
        cursor += n
    return tables


def decode_slots(tables, contexts, block_size: int):
    slots = np.empty(len(contexts), dtype=np.int32)
    for r, c in enumerate(contexts):
        pos = int(c) - 1
        slots[r] = tables[r, pos // block_size] * block_size + pos % block_size
    return slots


def make_decode_batch(
    *,
    num_seqs: int,
    ctx_lo: int,
    ctx_hi: int,
    pool_blocks: int,
    block_size: int = 16,
    num_q_heads: int,
    num_kv_heads: int,
    head_dim: int,
    seed: int = 0,
    draw_pools: bool = True,
    table_width: int | None = None,
) -> DecodeBatch:
    rng = np.random.default_rng(seed)
    contexts = rng.integers(ctx_lo, ctx_hi + 1, size=num_seqs).astype(np.int32)
    tables = draw_tables(rng, contexts, pool_blocks, block_size, table_width)
    batch = DecodeBatch(
        context_lens=contexts,
        block_tables=tables,
        slots=decode_slots(tables, contexts, block_size),
        block_size=block_size,
        pool_blocks=pool_blocks,
        meta=dict(seed=seed, num_q_heads=num_q_heads, num_kv_heads=num_kv_heads,
                  head_dim=head_dim),
    )
    batch.query = rng.standard_normal((num_seqs, num_q_heads, head_dim), dtype=np.float32)
    if draw_pools:
        pool_shape = (pool_blocks, block_size, num_kv_heads, head_dim)
        batch.key_pool = rng.standard_normal(pool_shape, dtype=np.float32)
        batch.value_pool = rng.standard_normal(pool_shape, dtype=np.float32)
        kv_shape = (num_seqs, num_kv_heads, head_dim)
        batch.new_keys = rng.standard_normal(kv_shape, dtype=np.float32)
        batch.new_values = rng.standard_normal(kv_shape, dtype=np.float32)
    return batch


@dataclass
class PrefillBatch:
    """A mixed prefill + decode step: varlen queries over paged caches."""

    q_lens: np.ndarray  # int32 [R]
    context_lens: np.ndarray  # int32 [R] (includes this step's rows)
    block_tables: np.ndarray  # int32 [R, W]
    cu_seqlens_q: np.ndarray  # int32 [R + 1]
    cu_seqlens_k: np.ndarray  # int32 [R + 1]
    block_size: int
    pool_blocks: int
    shared_blocks: int = 0


def make_mixed_prefill_batch(
    *,
    num_prefill: int = 8,
    chunk: int = 512,
    prefix_hi: int = 3072,
    shared_prefix: int = 1024,
    num_decode: int = 24,
    decode_lo: int = 256,
    decode_hi: int = 2048,
    pool_blocks: int = 65536,
    block_size: int = 16,
    seed: int = 0,
) -> PrefillBatch:
    """8 prefill chunks of 512 on prefixes U[0,3072] plus 24 decode rows.

    The first ``min(P_r, shared_prefix)`` prefix tokens, floored to whole
    blocks, map to the same block ids for every prefill request (prefix reuse
    shares only full blocks, microinfer/engine/blockmanager.py:144-181).
    """
    rng = np.random.default_rng(seed)
    prefixes = rng.integers(0, prefix_hi + 1, size=num_prefill)
    decode_ctx = rng.integers(decode_lo, decode_hi + 1, size=num_decode)
    q_lens = np.concatenate([np.full(num_prefill, chunk), np.ones(num_decode)]).astype(np.int32)
    contexts = np.concatenate([prefixes + chunk, decode_ctx]).astype(np.int32)
    perm = rng.permutation(pool_blocks)
    shared_n = shared_prefix // block_size
    shared_ids = perm[:shared_n]
    cursor = shared_n
    need = [(int(c) + block_size - 1) // block_size for c in contexts]
    tables = np.full((len(contexts), max(need)), -1, dtype=np.int32)
    for r, n in enumerate(need):
        reuse = min(int(prefixes[r]), shared_prefix) // block_size if r < num_prefill else 0
        tables[r, :reuse] = shared_ids[:reuse]
        fresh = n - reuse
        tables[r, reuse:n] = perm[cursor : cursor + fresh]
        cursor += fresh
    if cursor > pool_blocks:
        raise ValueError("pool too small")
    cu_q = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(contexts)]).astype(np.int32)
    return PrefillBatch(q_lens, contexts, tables, cu_q, cu_k, block_size, pool_blocks, shared_n)


# ---------------------------------------------------------------------------
# Algorithmic work per call (what a roofline is measured against).
# ---------------------------------------------------------------------------
def decode_bytes(contexts, *, num_q_heads, num_kv_heads, head_dim, elem_bytes, block_size,
                 with_append: bool = True) -> int:
    """HBM bytes one decode layer call must move at minimum.

    K and V rows read once (GQA groups share them) + Q read + O written +
    (append: new K/V read and written) + block-table entries + lens/slots.
    """
    contexts = np.asarray(contexts, dtype=np.int64)
    r = len(contexts)
    kv = int(contexts.sum()) * num_kv_heads * head_dim * 2 * elem_bytes
    qo = 2 * r * num_q_heads * head_dim * elem_bytes
    append = 2 * r * num_kv_heads * head_dim * 2 * elem_bytes if with_append else 0
    tables = int(((contexts + block_size - 1) // block_size).sum()) * 4
    return kv + qo + append + tables + 8 * r


def prefill_flops(q_lens, contexts, *, num_q_heads, head_dim) -> int:
    """Unmasked attention FLOPs: 4*Hq*D per (query, visible key) pair."""
    total = 0
    for q, c in zip(np.asarray(q_lens, dtype=np.int64), np.asarray(contexts, dtype=np.int64)):
        prefix = c - q
        total += 4 * num_q_heads * head_dim * (q * prefix + q * (q + 1) // 2)
    return int(total)


# The engine workload: random-init Qwen3-0.6B serving 64 requests of 128
# uniform-random prompt ids that arrive together, greedy, 16 output tokens
# each (EOS ignored); block 16, 4096 blocks, decode replayed from hipGraph
# buckets, mixed (decode-first) batches, max_num_seqs 64,
# max_num_batched_tokens 4096, max_num_prefill_tokens 512 -- the limits of
# the reference's published online run (docs/p4.md:172-176).
ENGINE_REQUESTS = 64
ENGINE_PROMPT_LEN = 128
ENGINE_OUTPUT_LEN = 16
ENGINE_NUM_BLOCKS = 4096
ENGINE_BLOCK_SIZE = 16


def engine_config(**overrides):
    from microinfer_amd.engine.config import EngineConfig

    values = dict(max_num_seqs=64, max_num_batched_tokens=4096, max_num_prefill_tokens=512,
                  max_model_len=4096, use_cuda_graph=True, mixed_batch=True)
    values.update(overrides)
    return EngineConfig(**values)


def engine_prompts(seed: int, vocab_size: int, requests: int = ENGINE_REQUESTS,
                   prompt_len: int = ENGINE_PROMPT_LEN) -> list[list[int]]:
    """One batch of the engine workload: ``requests`` prompts of uniform-random
    ids in [0, vocab_size), drawn one request after another from PCG64(seed)."""
    rng = np.random.default_rng(seed)
    return [rng.integers(0, vocab_size, prompt_len).tolist() for _ in range(requests)]


def engine_sampling():
    from microinfer_amd.engine.config import SampleParameter

    return SampleParameter(max_tokens=ENGINE_OUTPUT_LEN, ignore_eos=True, greedy=True)

"""KV-cache block ownership with prefix caching.

Mirrors ``Block`` / ``BlockManager`` (microinfer/engine/blockmanager.py:9-242):
the same public state (``blocks``, ``hash_to_block_id``, ``free_block_ids``,
``used_block_ids``, per-block ``ref_count`` / ``hash`` / ``token_ids``) and
the same rules, which the reference's tests pin
(tests/engine/test_blockmanager.py):

* a full block is identified by a 64-bit xxh64 chain hash -- the previous
  block's hash (8 bytes, little endian) then the block's token ids as int64
  -- and a hash hit is trusted only if the cached tokens are equal;
* a sequence's last block is never taken from the cache, so a partial block
  never exposes tokens beyond the sequence's length;
* freed blocks keep their KV and hash until reused; reuse takes the least
  recently used free block (a prefix lookup refreshes a block);
* hashes are published only for blocks completed by computed tokens
  (``hash_blocks``), never at allocation.

Here the free pool is one insertion-ordered dict (least recently used first):
touching a free block moves it to the end, so taking the oldest is O(1)
without the reference's lazily rebuilt heap.
"""

from __future__ import annotations

import numpy as np
import xxhash

from microinfer_amd.engine.sequence import Sequence


class Block:
    __slots__ = ("block_id", "ref_count", "hash", "token_ids")

    def __init__(self, block_id: int):
        self.block_id = block_id
        self.ref_count = 0
        self.hash = -1
        self.token_ids: list[int] = []

    def update(self, hash: int, token_ids: list[int]) -> None:  # noqa: A002
        self.hash = hash
        self.token_ids = token_ids

    def reset(self) -> None:
        """Fresh ownership by one sequence, no cached content."""
        self.ref_count = 1
        self.hash = -1
        self.token_ids = []


class BlockManager:
    def __init__(self, num_blocks: int, block_size: int):
        if type(num_blocks) is not int or type(block_size) is not int \
                or num_blocks <= 0 or block_size <= 0:
            raise ValueError("num_blocks and block_size must be positive integers")
        self.block_size = block_size
        self.blocks = [Block(i) for i in range(num_blocks)]
        self.hash_to_block_id: dict[int, int] = {}
        self._free: dict[int, None] = dict.fromkeys(range(num_blocks))  # LRU first
        self._published: dict[int, set[int]] = {}  # block id -> hashes it published
        self.used_block_ids: set[int] = set()
        self.prefix_cache_hit_tokens = 0
        self.prefix_cache_hit_blocks = 0
        self.prefix_cache_evictions = 0

    @property
    def free_block_ids(self):
        """Read-only view of the free block ids."""
        return self._free.keys()

    @classmethod
    def compute_hash(cls, token_ids: list[int], prefix: int = -1) -> int:
        h = xxhash.xxh64()
        if prefix != -1:
            h.update(prefix.to_bytes(8, "little"))
        h.update(np.asarray(token_ids, dtype=np.int64).tobytes())
        return h.intdigest()

    def stats(self) -> dict:
        total, used = len(self.blocks), len(self.used_block_ids)
        return {
            "num_blocks": total,
            "used_blocks": used,
            "free_blocks": len(self._free),
            "kv_utilization": used / total,
            "prefix_cache_entries": len(self.hash_to_block_id),
            "prefix_cache_hit_tokens": self.prefix_cache_hit_tokens,
            "prefix_cache_hit_blocks": self.prefix_cache_hit_blocks,
            "prefix_cache_evictions": self.prefix_cache_evictions,
        }

    # -- free pool ---------------------------------------------------------
    def _refresh(self, block_id: int) -> None:
        """Mark a block as just used: a free block moves to the young end."""
        if block_id in self._free:
            del self._free[block_id]
            self._free[block_id] = None

    def _take(self, block_id: int) -> None:
        del self._free[block_id]
        self.used_block_ids.add(block_id)

    def _release(self, block_id: int) -> None:
        block = self.blocks[block_id]
        block.ref_count -= 1
        if block.ref_count == 0:  # KV and hash stay until the block is reused
            self.used_block_ids.remove(block_id)
            self._free[block_id] = None

    def _forget(self, block_id: int) -> None:
        """Drop the hash entries that still point at a block being reused."""
        hashes = self._published.pop(block_id, set())
        if self.blocks[block_id].hash != -1:
            hashes.add(self.blocks[block_id].hash)
        for h in hashes:
            if self.hash_to_block_id.get(h) == block_id:
                del self.hash_to_block_id[h]

    def _allocate_block(self) -> int:
        if not self._free:
            raise RuntimeError("KV cache has no free blocks")
        block_id = next(iter(self._free))
        self._take(block_id)
        block = self.blocks[block_id]
        if block.token_ids:
            self.prefix_cache_evictions += 1
        self._forget(block_id)
        block.reset()
        return block_id

    # -- prefix lookup and allocation ----------------------------------------
    def _cached_prefix(self, seq: Sequence):
        """Yield (block id, hash) of the leading full blocks found in the
        cache, excluding the last block of the sequence."""
        prefix = -1
        for i in range(seq.num_blocks - 1):
            tokens = seq.block(i)
            h = self.compute_hash(tokens, prefix)
            block_id = self.hash_to_block_id.get(h)
            if block_id is None or self.blocks[block_id].token_ids != tokens:
                return
            yield block_id, h
            prefix = h

    def can_allocate(self, seq: Sequence) -> int:
        """Number of leading blocks the cache can supply, or -1 if the pool
        cannot hold the rest. Refreshes the blocks it finds."""
        reused = free_hits = 0
        for block_id, _ in self._cached_prefix(seq):
            reused += 1
            free_hits += block_id in self._free
            self._refresh(block_id)
        # A free cache hit leaves the free pool too, so it is not capacity.
        if seq.num_blocks - reused > len(self._free) - free_hits:
            return -1
        return reused

    def allocate(self, seq: Sequence, num_cached_blocks: int) -> None:
        """Give the sequence its cached prefix blocks and fresh blocks for the
        rest. Fresh blocks record their would-be hash, not yet published."""
        self.prefix_cache_hit_blocks += num_cached_blocks
        self.prefix_cache_hit_tokens += num_cached_blocks * self.block_size
        seq.num_cached_tokens = num_cached_blocks * self.block_size
        prefix = -1
        for i in range(seq.num_blocks):
            tokens = seq.block(i)
            h = self.compute_hash(tokens, prefix)
            prefix = h
            if i < num_cached_blocks:
                block_id = self.hash_to_block_id[h]
                if block_id in self._free:
                    self._take(block_id)
                self.blocks[block_id].ref_count += 1
                self._refresh(block_id)
            else:
                block_id = self._allocate_block()
                self.blocks[block_id].update(h, tokens)
            seq.block_table.append(block_id)

    def deallocate(self, seq: Sequence) -> None:
        seq.num_cached_tokens = 0
        for block_id in seq.block_table:
            self._release(block_id)
        seq.block_table.clear()

    def trim(self, seq: Sequence) -> None:
        """Release table entries beyond the sequence's current length."""
        while len(seq.block_table) > seq.num_blocks:
            self._release(seq.block_table.pop())

    def can_append(self, seq: Sequence) -> bool:
        return len(self._free) >= max(0, seq.num_blocks - len(seq.block_table))

    def may_append(self, seq: Sequence) -> None:
        if not self.can_append(seq):
            raise ValueError("insufficient cache blocks")
        while len(seq.block_table) < seq.num_blocks:
            seq.block_table.append(self._allocate_block())

    def hash_blocks(self, seq: Sequence) -> None:
        """Publish the blocks that the scheduled tokens complete."""
        first = seq.num_cached_tokens // self.block_size
        last = (seq.num_cached_tokens + seq.num_scheduled_tokens) // self.block_size
        prefix = self.blocks[seq.block_table[first - 1]].hash if first else -1
        for i in range(first, last):
            tokens = seq.block(i)
            prefix = self.compute_hash(tokens, prefix)
            block_id = seq.block_table[i]
            self.hash_to_block_id[prefix] = block_id
            self._published.setdefault(block_id, set()).add(prefix)
            self.blocks[block_id].update(prefix, tokens)

    def reset_prefix_cache(self) -> None:
        """Forget every cached prefix; only while no block is in use."""
        if self.used_block_ids:
            raise RuntimeError("cannot reset prefix cache while blocks are in use")
        self.hash_to_block_id.clear()
        self._published.clear()
        for block in self.blocks:
            block.hash, block.token_ids = -1, []
        self.prefix_cache_hit_tokens = self.prefix_cache_hit_blocks = 0
        self.prefix_cache_evictions = 0

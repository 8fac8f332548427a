"""KV-cached paged Qwen3 forward on the host (test infrastructure and the
engine workload's CPU baseline only).

TEST INFRASTRUCTURE ONLY: imported by ``tests/`` and by the bench's
``cpu_baseline`` leg, never by the product package.

``HostPagedRunner`` has the ``run(seqs, is_prefill) -> tokens`` contract of
the engine's model runner, so ``LLMEngine`` drives it with the product's own
``Scheduler`` and ``BlockManager``: the same steps, chunks, block tables and
slots as on the GPU. Each step follows the reference's runner and model on
its CPU path, in float32:

* step metadata as ``ModelRunner.prepare_prefill`` / ``prepare_decode``
  build it (microinfer/runner.py:298-385; ``oracle.step_metadata``);
* per layer (microinfer/layer/transformer.py:186-252): RMSNorm carrying the
  residual sum (norm.py:26-35), the fused QKV product, Q/K RMSNorm + RoPE
  and the append of K/V into a paged float32 cache at the step's slots
  (``oracle.qk_norm_rope.qk_norm_rope_append``, kv_cache.py:52-79), paged
  causal GQA attention over the cache (``oracle.paged_attention.
  paged_attention_reference``, layer/paged_attention.py:22-67), the output
  product, the second norm and SwiGLU (transformer.py:90-98);
* the final norm, the vocabulary product for each request's last row, and
  ``argmax`` (runner.py:240, sampler.py:44-45).

Greedy requests only. Pinned (tests/test_oracle_host_runner.py) by the dense
oracle: through the engine, with chunked prefill, mixed steps and prefix
reuse, every greedy token equals ``oracle.qwen3_dense``'s teacher-forced
choice.
"""

from __future__ import annotations

import numpy as np

from oracle.greedy import greedy_argmax
from oracle.paged_attention import paged_attention_reference
from oracle.qk_norm_rope import qk_norm_rope_append, rms_norm, rope_tables
from oracle.step_metadata import decode_rows, prefill_rows


class HostPagedRunner:
    def __init__(self, weights: dict, config, num_blocks: int, block_size: int):
        self.w = weights
        self.c = config
        self.block_size = block_size
        shape = (config.num_hidden_layer, num_blocks, block_size, config.num_kv_head,
                 config.head_dim)
        # np.zeros maps untouched pages lazily: only written blocks cost memory.
        self.key_cache = np.zeros(shape, dtype=np.float32)
        self.value_cache = np.zeros(shape, dtype=np.float32)
        self.cos, self.sin = rope_tables(config.max_pos_embed, config.head_dim,
                                         config.rope_base)

    def _norm(self, x, residual, weight):
        combined = x if residual is None else x + residual
        return rms_norm(combined, weight, self.c.norm_eps, "f32"), combined

    def run(self, seqs, is_prefill: bool) -> list[int]:
        if any(not s.greedy for s in seqs):
            raise ValueError("the host runner samples greedily only")
        if is_prefill:
            meta = prefill_rows(seqs, self.block_size)
            cu_q = meta["cu_seqlens_q"]
            contexts = np.diff(meta["cu_seqlens_k"])
        else:
            meta = decode_rows(seqs, self.block_size)
            cu_q = np.arange(len(seqs) + 1, dtype=np.int32)
            contexts = meta["context_lens"]
        width = max(len(s.block_table) for s in seqs)
        tables = np.full((len(seqs), max(width, 1)), -1, dtype=np.int32)
        for i, s in enumerate(seqs):
            tables[i, :len(s.block_table)] = s.block_table
        logits = self.forward(meta["input_ids"], meta["positions"], meta["slot_mapping"],
                              cu_q, contexts, tables)
        return [int(t) for t in greedy_argmax(logits)]

    def forward(self, ids, positions, slots, cu_q, contexts, tables) -> np.ndarray:
        """Logits ``[R, vocab]`` of each request's last scheduled row."""
        c, w = self.c, self.w
        t, d = len(ids), c.head_dim
        hidden = w["embedding"][np.asarray(ids, dtype=np.int64)].astype(np.float32)
        residual = None
        scale = 1.0 / np.sqrt(d)
        for i, layer in enumerate(w["layers"]):
            x, residual = self._norm(hidden, residual, layer["pre_norm"])
            qkv = x @ layer["qkv"].T
            q, _ = qk_norm_rope_append(
                qkv, layer["q_norm"], layer["k_norm"], c.norm_eps, self.cos, self.sin,
                positions, slots, self.key_cache[i], self.value_cache[i],
                num_q_heads=c.num_q_head, num_kv_heads=c.num_kv_head, head_dim=d,
                interleaved=c.rope_interleaved, dtype="f32")
            attn = paged_attention_reference(q, self.key_cache[i], self.value_cache[i], tables,
                                             contexts, cu_q, scale=scale)
            hidden = attn.reshape(t, c.num_q_head * d) @ layer["out"].T
            x, residual = self._norm(hidden, residual, layer["post_norm"])
            gate, up = np.split(x @ layer["gate_up"].T, 2, axis=-1)
            hidden = (gate / (np.float32(1) + np.exp(-gate)) * up) @ layer["down"].T
        last = np.asarray(cu_q[1:], dtype=np.int64) - 1
        final, _ = self._norm(hidden[last], residual[last], w["final_norm"])
        return final @ w["lm_head"].T

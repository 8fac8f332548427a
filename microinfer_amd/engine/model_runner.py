"""Runs one scheduled step of the model and returns the sampled tokens.

Mirrors ``ModelRunner.run`` / ``run_model`` / ``_run_decode``
(microinfer/runner.py:555-626): prefill steps build their metadata on the
device and run eagerly; decode steps replay the smallest captured hipGraph
bucket that holds the batch (greedy tokens selected inside the graph) or run
eagerly when no bucket fits or graphs are off; greedy rows take the argmax,
the others the temperature sampler, mixed per row as the reference does.

The KV pool has one block more than the block manager hands out: the pad
rows of graph buckets write their K/V there. With ``EngineConfig.debug_mode``
each step's metadata is validated before launch (``runner.validate_step``).
"""

from __future__ import annotations

import torch

from microinfer_amd.engine.config import EngineConfig
from microinfer_amd.layer.hip_sampler import Sampler, greedy_argmax
from microinfer_amd.runner import DecodeGraphRunner, StepMetadataBuilder
from microinfer_amd.worker.kv_cache import KVCache


class ModelRunner:
    def __init__(self, model, config: EngineConfig, *, num_blocks: int, block_size: int,
                 layout: str = "paired"):
        c = model.config
        self.model, self.config = model, config
        self.num_blocks, self.block_size = num_blocks, block_size
        self.kv_cache = KVCache(c.num_hidden_layer, num_blocks + 1, block_size, c.num_kv_head,
                                c.head_dim, dtype=model.dtype, device=model.device,
                                layout=layout)
        model.bind_caches([self.kv_cache.layer(i) for i in range(c.num_hidden_layer)])
        self.builder = StepMetadataBuilder(block_size, model.device, pad_block_id=num_blocks,
                                           debug_mode=config.debug_mode, num_blocks=num_blocks,
                                           max_pos_embed=c.max_pos_embed,
                                           vocab_size=c.vocab_size)
        self.sampler = Sampler()
        self.graphs = None
        if config.use_cuda_graph:
            self.graphs = DecodeGraphRunner(self.builder, self.run_model,
                                            max_num_seqs=config.max_num_seqs,
                                            table_width=num_blocks + 1, greedy=True)

    def run_model(self, input_ids, positions, metadata):
        return self.model.compute_logits(self.model.forward(input_ids, positions, metadata),
                                         metadata)

    @torch.inference_mode()
    def run(self, seqs, is_prefill: bool) -> list[int]:
        if not seqs:
            return []
        greedy_tokens = None
        if is_prefill:
            logits = self.run_model(*self.builder.prepare_prefill(seqs))
        else:
            replayed = self.graphs.run(seqs) if self.graphs is not None else None
            if replayed is not None:
                logits, greedy_tokens = replayed
            else:
                logits = self.run_model(*self.builder.prepare_decode(seqs))
        flags = [seq.greedy for seq in seqs]
        if all(flags):
            tokens = greedy_tokens if greedy_tokens is not None else greedy_argmax(logits)
        else:
            temperatures = torch.tensor([seq.temperature for seq in seqs],
                                        dtype=torch.float32, device=logits.device)
            tokens = self.sampler(logits, temperatures)
            if any(flags):
                greedy = greedy_tokens if greedy_tokens is not None else greedy_argmax(logits)
                mask = torch.tensor(flags, dtype=torch.bool, device=logits.device)
                tokens = torch.where(mask, greedy, tokens)
        return tokens.tolist()

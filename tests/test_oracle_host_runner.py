"""Pin of the host paged runner (oracle/qwen3_paged_host.py), CPU only.

Driven by the product's Scheduler and BlockManager through LLMEngine, with
chunked prefill, mixed decode + prefill steps, prefix-cache reuse and
preemption, every greedy token it produces must equal the dense oracle's
teacher-forced choice (oracle/qwen3_dense.py, float64 products, full
recompute without any cache). A wrong slot, a stale cache row, a mis-ordered
residual or a wrong RoPE position changes tokens.
"""

from types import SimpleNamespace

import numpy as np
import pytest

from microinfer_amd.engine.blockmanager import BlockManager
from microinfer_amd.engine.config import EngineConfig, SampleParameter
from microinfer_amd.engine.llm_engine import LLMEngine
from microinfer_amd.engine.scheduler import Scheduler
from oracle.qwen3_dense import teacher_forced, weights_f64
from oracle.qwen3_paged_host import HostPagedRunner
from tests.test_oracle_qwen3_dense import make_weights

CFG = SimpleNamespace(vocab_size=96, hidden_dim=64, norm_eps=1e-6, MLP_inter_dim=96,
                      num_q_head=4, num_kv_head=2, head_dim=16, num_hidden_layer=2,
                      rope_base=10000.0, rope_interleaved=False, max_pos_embed=256)
GREEDY = SampleParameter(max_tokens=6, greedy=True)


def make_engine(weights, *, num_blocks=32, block_size=4, **limits):
    values = dict(max_num_seqs=4, max_num_batched_tokens=12, max_num_prefill_tokens=8,
                  max_model_len=128)
    values.update(limits)
    config = EngineConfig(**values)
    runner = HostPagedRunner(weights, CFG, num_blocks, block_size)
    return LLMEngine(Scheduler(config, BlockManager(num_blocks, block_size)), runner)


def check(weights, prompts, outputs):
    wide = weights_f64(weights)
    checked = 0
    for prompt, got in zip(prompts, outputs):
        want, gaps = teacher_forced(wide, CFG, prompt, got)
        for g, w, gap in zip(got, want, gaps):
            assert g == w or gap < 1e-4
            checked += 1
    return checked


def prompts(seed, lengths):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, CFG.vocab_size, n).tolist() for n in lengths]


@pytest.mark.parametrize("mixed", [True, False])
def test_host_runner_matches_dense_oracle(mixed, sequence_cls):
    weights = make_weights(CFG, seed=11)
    engine = make_engine(weights, mixed_batch=mixed)
    batch = prompts(1, [1, 5, 9, 14, 3])
    out = engine.generate(batch, GREEDY)
    assert check(weights, batch, out) == 30
    stats = engine.stats()
    assert stats["used_blocks"] == 0
    if mixed:
        assert stats["num_mixed_steps"] > 0


def test_host_runner_prefix_reuse_and_preemption(sequence_cls):
    weights = make_weights(CFG, seed=12)
    engine = make_engine(weights)
    base = prompts(2, [13])[0]
    engine.generate([base], GREEDY)
    follow = [base[:8] + [1, 2, 3], list(base)]
    out = engine.generate(follow, GREEDY)
    assert engine.stats()["prefix_cache_hit_blocks"] >= 2
    assert check(weights, follow, out) == 12
    tight = make_engine(weights, num_blocks=7, max_num_batched_tokens=32,
                        max_num_prefill_tokens=32)
    batch = prompts(3, [9, 10, 8])
    out = tight.generate(batch, SampleParameter(max_tokens=5, greedy=True))
    assert tight.stats()["num_preemptions"] > 0
    assert check(weights, batch, out) == 15


def test_host_runner_rejects_sampled_rows(sequence_cls):
    weights = make_weights(CFG, seed=13)
    engine = make_engine(weights)
    with pytest.raises(ValueError, match="greedily"):
        engine.generate([[1, 2]], SampleParameter(max_tokens=2))

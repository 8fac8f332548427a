"""The engine end to end on the device: greedy tokens against the dense
oracle (oracle/qwen3_dense.py).

A small random Qwen3 (2 layers, 4 Q / 2 KV heads, head_dim 32, float32) runs
through the engine -- scheduler, block manager, device-built metadata, the
fused Q/K norm + RoPE + append, paged/varlen attention, graph-captured decode
with the in-graph argmax -- and every generated token must equal the token
the oracle chooses by recomputing the whole sequence densely; the two may
part only at a position whose top-2 logit gap in the oracle is below the
tolerance (only there may other rounding flip the choice), after which the
continuations differ. Chunked prefill, mixed steps, prefix-cache reuse
and preemption must not change any token. A Qwen3-0.6B-shaped bfloat16 layer
stack (MFMA prefill), and the full 28-layer Qwen3-0.6B of the engine
workload, are checked the same way with a wider gap tolerance.
"""

import numpy as np
import pytest
import torch

from microinfer_amd.engine.blockmanager import BlockManager
from microinfer_amd.engine.config import EngineConfig, SampleParameter
from microinfer_amd.engine.llm_engine import LLMEngine
from microinfer_amd.engine.model import QwenConfig, Qwen3Model
from microinfer_amd.engine.model_runner import ModelRunner
from microinfer_amd.engine.scheduler import Scheduler
from microinfer_amd.engine.sequence import Sequence
from oracle.qwen3_dense import greedy_generate

pytestmark = pytest.mark.gpu

TINY = QwenConfig(vocab_size=512, hidden_dim=128, MLP_inter_dim=256, num_q_head=4,
                  num_kv_head=2, head_dim=32, num_hidden_layer=2, max_pos_embed=512)
GREEDY = SampleParameter(max_tokens=6, greedy=True)


def make_engine(model, *, num_blocks=64, block_size=16, **limits):
    values = dict(max_num_seqs=8, max_num_batched_tokens=24, max_num_prefill_tokens=16,
                  max_model_len=256, use_cuda_graph=True)
    values.update(limits)
    config = EngineConfig(**values)
    runner = ModelRunner(model, config, num_blocks=num_blocks, block_size=block_size)
    return LLMEngine(Scheduler(config, BlockManager(num_blocks, block_size)), runner)


def prompts(seed, lengths, vocab=512):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, vocab, n).tolist() for n in lengths]


def check_against_oracle(model, prompt_list, outputs, max_tokens, gap_tol):
    weights = model.host_weights()
    compared = 0
    for prompt, got in zip(prompt_list, outputs):
        want, gaps = greedy_generate(weights, model.config, prompt, max_tokens)
        assert len(got) == len(want)
        for i, (g, w, gap) in enumerate(zip(got, want, gaps)):
            if g != w:
                # Only a near-tie may flip under other rounding; the two
                # continuations then legitimately differ.
                assert gap < gap_tol, f"prompt len {len(prompt)}: token {i} is {g}, oracle {w}"
                break
            compared += 1
    return compared


@pytest.fixture(scope="module")
def tiny_model():
    return Qwen3Model(TINY, dtype=torch.float32, device="cuda", seed=0, init_std=0.1)


@pytest.mark.parametrize("graph", [True, False])
@pytest.mark.parametrize("mixed", [True, False])
def test_greedy_tokens_match_dense_oracle(tiny_model, graph, mixed):
    engine = make_engine(tiny_model, use_cuda_graph=graph, mixed_batch=mixed)
    batch = prompts(1, [1, 7, 16, 17, 33, 40])
    out = engine.generate(batch, GREEDY)
    compared = check_against_oracle(tiny_model, batch, out, 6, 1e-4)
    assert compared >= 30
    stats = engine.stats()
    assert stats["num_steps"] > 6 and stats["used_blocks"] == 0
    if mixed:
        assert stats["num_mixed_steps"] > 0


def test_prefix_cache_reuse_keeps_tokens(tiny_model):
    engine = make_engine(tiny_model)
    base = prompts(2, [40])[0]
    engine.generate([base], GREEDY)
    follow = [base[:32] + prompts(3, [5])[0], list(base)]
    out = engine.generate(follow, GREEDY)
    assert engine.stats()["prefix_cache_hit_blocks"] >= 4
    assert check_against_oracle(tiny_model, follow, out, 6, 1e-4) >= 10


def test_preemption_keeps_tokens(tiny_model):
    engine = make_engine(tiny_model, num_blocks=6, max_num_batched_tokens=64,
                         max_num_prefill_tokens=64)
    batch = prompts(4, [30, 31, 29])
    params = SampleParameter(max_tokens=12, greedy=True)
    out = engine.generate(batch, params)
    assert engine.stats()["num_preemptions"] > 0
    assert check_against_oracle(tiny_model, batch, out, 12, 1e-4) >= 20


def test_sampled_and_greedy_rows_in_one_batch(tiny_model):
    engine = make_engine(tiny_model)
    batch = prompts(5, [9, 12, 20])
    params = [GREEDY, SampleParameter(temperature=0.7, max_tokens=6), GREEDY]
    out = engine.generate(batch, params)
    assert all(len(o) == 6 and all(0 <= t < TINY.vocab_size for t in o) for o in out)
    greedy = [batch[0], batch[2]]
    assert check_against_oracle(tiny_model, greedy, [out[0], out[2]], 6, 1e-4) >= 8


def test_bf16_qwen3_layers_match_oracle():
    config = QwenConfig(vocab_size=4096, hidden_dim=1024, MLP_inter_dim=3072, num_q_head=16,
                        num_kv_head=8, head_dim=128, num_hidden_layer=2, max_pos_embed=1024)
    model = Qwen3Model(config, dtype=torch.bfloat16, device="cuda", seed=7, init_std=0.05)
    engine = make_engine(model, max_num_batched_tokens=96, max_num_prefill_tokens=64)
    batch = prompts(6, [5, 64, 100, 17, 33, 80], vocab=4096)
    out = engine.generate(batch, SampleParameter(max_tokens=6, greedy=True))
    # bf16 weights are exact in the oracle; activations round at every
    # product (logit spread about 1.6), so a flip is allowed only where the
    # oracle's top two logits are within 0.1.
    assert check_against_oracle(model, batch, out, 6, 0.1) >= 12


def test_engine_rejects_requests_beyond_capacity(tiny_model):
    engine = make_engine(tiny_model, debug_mode=True, max_model_len=32)
    with pytest.raises(ValueError):
        engine.add_request(Sequence(list(range(40)), GREEDY))


def test_qwen3_06b_engine_matches_oracle():
    # The engine workload's model itself: Qwen3-0.6B dimensions (28 layers,
    # vocabulary 151936), bf16, N(0, 0.02) weights, seed 0; four prompts of
    # the workload's kind, four greedy tokens each. The oracle recomputes
    # every sequence densely on the host (about 4 s per prompt).
    model = Qwen3Model(QwenConfig(), dtype=torch.bfloat16, device="cuda", seed=0)
    engine = make_engine(model, num_blocks=256, max_num_batched_tokens=512,
                         max_num_prefill_tokens=512)
    batch = prompts(5, [128, 64, 17, 100], vocab=151936)
    out = engine.generate(batch, SampleParameter(max_tokens=4, greedy=True))
    assert check_against_oracle(model, batch, out, 4, 0.03) >= 12

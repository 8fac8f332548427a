"""The engine end to end on the device: greedy tokens against the dense
oracle (oracle/qwen3_dense.py), checked teacher-forced.

A small random Qwen3 (2 layers, 4 Q / 2 KV heads, head_dim 32, float32) runs
through the engine -- scheduler, block manager, device-built metadata, the
fused Q/K norm + RoPE + append, paged/varlen attention, graph-captured decode
with the in-graph argmax. For every request the oracle then runs ONE dense
forward over the prompt and the engine's own tokens, and every emitted token
must be the oracle's greedy choice at its position, or a token whose oracle
logit lies within the tolerance of the best one (a near-tie that other
rounding may flip); the positions after such a flip are still checked, on the
engine's path. Every position is counted, with no early exit. Chunked prefill, mixed steps, prefix-cache reuse and preemption must
not change any token. A Qwen3-0.6B-shaped bfloat16 layer stack (MFMA
prefill), the full 28-layer Qwen3-0.6B, and the engine workload itself (64
requests x 128 prompt ids -> 16 greedy tokens, 4096 blocks, graph decode,
mixed batches) are checked the same way with a wider tolerance.
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
from microinfer_amd.workloads import (ENGINE_BLOCK_SIZE, ENGINE_NUM_BLOCKS, ENGINE_OUTPUT_LEN,
                                      engine_config, engine_prompts, engine_sampling)
from oracle.qwen3_dense import token_deficits, weights_f64

pytestmark = pytest.mark.gpu

TINY = QwenConfig(vocab_size=512, hidden_dim=128, MLP_inter_dim=256, num_q_head=4,
                  num_kv_head=2, head_dim=32, num_hidden_layer=2, max_pos_embed=512)
GREEDY = SampleParameter(max_tokens=6, greedy=True)


# Full 28-layer Qwen3-0.6B in bf16: activations round at every product, so
# the engine's logits drift from the float64 oracle's by a few hundredths and
# near-ties flip with the order of float32 sums (the HIP projections flip
# one of 256 checked positions by 0.032 that hipBLASLt's keep). On this
# model the oracle's median top-1/top-2 gap is 0.075 and a row's logits
# spread with a standard deviation of 0.64 (measured on a 128-token prompt),
# so a wrong token sits tenths below the best, far outside this bound.
QWEN3_06B_TOLERANCE = 0.05


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


def check_against_oracle(model, prompt_list, outputs, max_tokens, tolerance):
    """Teacher-forced check of every emitted token; returns ``(checked,
    exact)``: how many positions were checked and at how many the engine's
    token IS the oracle's greedy choice. At each position the oracle's logit
    of the engine's token must be within ``tolerance`` of the oracle's best
    logit there: equal to its greedy choice, or a near-tie that other
    rounding may flip."""
    weights = weights_f64(model.host_weights())
    checked = exact = 0
    for prompt, got in zip(prompt_list, outputs):
        assert len(got) == max_tokens, f"prompt len {len(prompt)}: {len(got)} tokens"
        deficits = token_deficits(weights, model.config, prompt, got)
        for i, (tok, deficit) in enumerate(zip(got, deficits)):
            checked += 1
            exact += deficit == 0.0
            assert deficit <= tolerance, (f"prompt len {len(prompt)}: token {i} ({tok}) is "
                                          f"{deficit:.4g} below the oracle's best logit")
    print(f"teacher-forced: {exact} of {checked} tokens are the oracle's exact argmax")
    return checked, exact


@pytest.fixture(scope="module")
def tiny_model():
    return Qwen3Model(TINY, dtype=torch.float32, device="cuda", seed=0, init_std=0.1)


@pytest.mark.parametrize("graph", [True, False])
@pytest.mark.parametrize("mixed", [True, False])
def test_greedy_tokens_match_dense_oracle(tiny_model, graph, mixed):
    engine = make_engine(tiny_model, use_cuda_graph=graph, mixed_batch=mixed)
    batch = prompts(1, [1, 7, 16, 17, 33, 40])
    out = engine.generate(batch, GREEDY)
    assert check_against_oracle(tiny_model, batch, out, 6, 1e-4) == (36, 36)
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
    assert check_against_oracle(tiny_model, follow, out, 6, 1e-4) == (12, 12)


def test_preemption_keeps_tokens(tiny_model):
    engine = make_engine(tiny_model, num_blocks=6, max_num_batched_tokens=64,
                         max_num_prefill_tokens=64)
    batch = prompts(4, [30, 31, 29])
    params = SampleParameter(max_tokens=12, greedy=True)
    out = engine.generate(batch, params)
    assert engine.stats()["num_preemptions"] > 0
    assert check_against_oracle(tiny_model, batch, out, 12, 1e-4) == (36, 36)


def test_sampled_and_greedy_rows_in_one_batch(tiny_model):
    engine = make_engine(tiny_model)
    batch = prompts(5, [9, 12, 20])
    params = [GREEDY, SampleParameter(temperature=0.7, max_tokens=6), GREEDY]
    out = engine.generate(batch, params)
    assert all(len(o) == 6 and all(0 <= t < TINY.vocab_size for t in o) for o in out)
    greedy = [batch[0], batch[2]]
    assert check_against_oracle(tiny_model, greedy, [out[0], out[2]], 6, 1e-4) == (12, 12)


def test_bf16_qwen3_layers_match_oracle():
    config = QwenConfig(vocab_size=4096, hidden_dim=1024, MLP_inter_dim=3072, num_q_head=16,
                        num_kv_head=8, head_dim=128, num_hidden_layer=2, max_pos_embed=1024)
    model = Qwen3Model(config, dtype=torch.bfloat16, device="cuda", seed=7, init_std=0.05)
    engine = make_engine(model, max_num_batched_tokens=96, max_num_prefill_tokens=64)
    batch = prompts(6, [5, 64, 100, 17, 33, 80], vocab=4096)
    out = engine.generate(batch, SampleParameter(max_tokens=6, greedy=True))
    # bf16 weights are exact in the oracle; activations round at every
    # product (logit spread about 1.6), so a token may sit up to 0.1 below
    # the oracle's best logit.
    checked, exact = check_against_oracle(model, batch, out, 6, 0.1)
    assert checked == 36 and exact >= 34


def test_engine_rejects_requests_beyond_capacity(tiny_model):
    engine = make_engine(tiny_model, debug_mode=True, max_model_len=32)
    with pytest.raises(ValueError):
        engine.add_request(Sequence(list(range(40)), GREEDY))


def test_qwen3_06b_engine_matches_oracle():
    # The engine workload's model itself: Qwen3-0.6B dimensions (28 layers,
    # vocabulary 151936), bf16, N(0, 0.02) weights, seed 0; four prompts of
    # the workload's kind, four greedy tokens each, on a small cache.
    model = Qwen3Model(QwenConfig(), dtype=torch.bfloat16, device="cuda", seed=0)
    engine = make_engine(model, num_blocks=256, max_num_batched_tokens=512,
                         max_num_prefill_tokens=512)
    batch = prompts(5, [128, 64, 17, 100], vocab=151936)
    out = engine.generate(batch, SampleParameter(max_tokens=4, greedy=True))
    checked, exact = check_against_oracle(model, batch, out, 4, QWEN3_06B_TOLERANCE)
    assert checked == 16 and exact >= 15


def test_engine_workload_matches_oracle_teacher_forced():
    # The engine workload exactly as the bench runs it: random-init
    # Qwen3-0.6B (bf16, seed 0), 64 requests x 128 uniform-random prompt ids
    # (batch seed 0) arriving together, 16 greedy tokens each, block 16,
    # 4096 blocks, graph-captured decode, mixed batches. Every 4th request
    # (16 of 64, 256 generated tokens) is checked teacher-forced against the
    # dense oracle; all 64 must finish with 16 tokens.
    model = Qwen3Model(QwenConfig(), dtype=torch.bfloat16, device="cuda", seed=0)
    config = engine_config()
    runner = ModelRunner(model, config, num_blocks=ENGINE_NUM_BLOCKS,
                         block_size=ENGINE_BLOCK_SIZE)
    engine = LLMEngine(Scheduler(config, BlockManager(ENGINE_NUM_BLOCKS, ENGINE_BLOCK_SIZE)),
                       runner)
    batch = engine_prompts(0, model.config.vocab_size)
    out = engine.generate(batch, engine_sampling())
    assert all(len(o) == ENGINE_OUTPUT_LEN for o in out)
    stats = engine.stats()
    assert stats["num_mixed_steps"] + stats["num_decode_steps"] >= ENGINE_OUTPUT_LEN - 1
    assert stats["used_blocks"] == 0
    picked = list(range(0, len(batch), 4))
    checked, exact = check_against_oracle(model, [batch[i] for i in picked],
                                          [out[i] for i in picked], ENGINE_OUTPUT_LEN,
                                          QWEN3_06B_TOLERANCE)
    assert checked == 16 * ENGINE_OUTPUT_LEN
    # Near-ties aside, the tokens ARE the oracle's greedy tokens: at least
    # 95 % of the 256 positions are its exact argmax.
    assert exact >= 0.95 * checked, f"only {exact} of {checked} exact"


def test_async_engine_on_a_side_stream_matches_generate(tiny_model):
    # Two requests admitted concurrently through the async frontend, whose
    # worker thread makes a side stream current: the HIP library reads the
    # stream at call time, so every kernel of every step lands on that
    # stream, and the tokens equal the synchronous engine's.
    import asyncio

    from microinfer_amd.engine.async_engine import AsyncEngine

    batch = prompts(8, [21, 9])
    expected = make_engine(tiny_model).generate(batch, GREEDY)
    side = torch.cuda.Stream()
    engine = make_engine(tiny_model)
    seen = []
    run = engine.model_runner.run

    def recording_run(seqs, is_prefill):
        seen.append(torch.cuda.current_stream() == side)
        return run(seqs, is_prefill)

    engine.model_runner.run = recording_run

    async def scenario():
        frontend = AsyncEngine(engine, stream=side)
        outs = await asyncio.gather(*(frontend.generate(p, GREEDY) for p in batch))
        await frontend.stop()
        return outs

    outs = asyncio.run(scenario())
    torch.cuda.synchronize()
    assert [list(o.token_ids) for o in outs] == expected
    assert seen and all(seen)
    assert check_against_oracle(tiny_model, batch, expected, 6, 1e-4) == (12, 12)


@pytest.mark.parametrize("graph", [True, False])
def test_debug_mode_validates_every_step_and_keeps_tokens(tiny_model, graph, monkeypatch):
    # EngineConfig.debug_mode: every prefill, eager decode and graph-bucket
    # decode step goes through runner.validate_step (microinfer/runner.py:
    # 387-528) before launch, and the tokens do not change.
    import microinfer_amd.runner as runner_module

    seen = []
    real = runner_module.validate_step

    def recording(seqs, input_ids, positions, metadata, is_prefill, **limits):
        seen.append(is_prefill)
        assert limits["num_blocks"] == 64 and limits["vocab_size"] == TINY.vocab_size
        return real(seqs, input_ids, positions, metadata, is_prefill, **limits)

    monkeypatch.setattr(runner_module, "validate_step", recording)
    batch = prompts(1, [1, 7, 16, 17, 33, 40])
    expected = make_engine(tiny_model, use_cuda_graph=graph).generate(batch, GREEDY)
    assert not seen
    engine = make_engine(tiny_model, use_cuda_graph=graph, debug_mode=True)
    assert engine.generate(batch, GREEDY) == expected
    assert True in seen and False in seen

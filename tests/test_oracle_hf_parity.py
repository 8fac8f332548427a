"""The dense Qwen3 oracle against an independent implementation, on the CPU.

Restates the reference's offline parity check (tests/integration/
test_hf_parity.py:17-113): a tiny random ``transformers.Qwen3ForCausalLM``
(eager attention, float32) is the reference, and ``oracle/qwen3_dense.py``
runs on the same weights, fused the way the product model stores them (Q/K/V
rows stacked into one projection, gate and up rows into another). Checked:

* dense logits of every position to 1e-5 absolute / 1e-4 relative, with the
  vocabulary head tied to the embedding (the reference's fixture) and untied
  (the reference model's default, config/config.py:21);
* greedy generation: the oracle's tokens equal the ones the transformers
  model picks by argmax of its last row, step by step;
* a prefix-sharing prompt (the reference's prefix-reuse case) gives the same
  last-row logits.

This pins the parts of the oracle that a shared misreading could otherwise
hide: the per-head Q/K norm before RoPE, the split-half rotation, the
residual carried through the norms, SwiGLU's gate/up order and the GQA head
map. Nothing here imports the product package.
"""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle.qwen3_dense import forward_logits, greedy_generate

transformers = pytest.importorskip("transformers")


def hf_pair(tie: bool, seed: int = 13):
    config = transformers.Qwen3Config(
        vocab_size=32, hidden_size=16, intermediate_size=32, num_hidden_layers=2,
        num_attention_heads=4, num_key_value_heads=2, head_dim=4,
        max_position_embeddings=64, rms_norm_eps=1e-6, tie_word_embeddings=tie,
        attention_dropout=0.0)
    config._attn_implementation = "eager"
    torch.manual_seed(seed)
    model = transformers.Qwen3ForCausalLM(config).eval()
    # The default initialisation leaves every norm weight at 1: perturb them
    # so that a norm applied in the wrong place changes the logits.
    gen = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("norm.weight"):
                p.add_(0.2 * torch.randn(p.shape, generator=gen))
    rope = config.to_dict().get("rope_parameters") or {}
    cfg = SimpleNamespace(
        vocab_size=config.vocab_size, hidden_dim=config.hidden_size,
        norm_eps=config.rms_norm_eps, MLP_inter_dim=config.intermediate_size,
        num_q_head=config.num_attention_heads, num_kv_head=config.num_key_value_heads,
        head_dim=config.head_dim, num_hidden_layer=config.num_hidden_layers,
        rope_base=float(rope.get("rope_theta", getattr(config, "rope_theta", 10000.0))),
        rope_interleaved=False)
    return model, cfg


def oracle_weights(model) -> dict:
    """The transformers parameters in the oracle's (product model's) layout."""
    sd = {k: v.detach().float().numpy() for k, v in model.state_dict().items()}
    layers = []
    for i in range(model.config.num_hidden_layers):
        p = f"model.layers.{i}."
        layers.append(dict(
            pre_norm=sd[p + "input_layernorm.weight"],
            qkv=np.concatenate([sd[p + "self_attn.q_proj.weight"],
                                sd[p + "self_attn.k_proj.weight"],
                                sd[p + "self_attn.v_proj.weight"]], axis=0),
            q_norm=sd[p + "self_attn.q_norm.weight"],
            k_norm=sd[p + "self_attn.k_norm.weight"],
            out=sd[p + "self_attn.o_proj.weight"],
            post_norm=sd[p + "post_attention_layernorm.weight"],
            gate_up=np.concatenate([sd[p + "mlp.gate_proj.weight"],
                                    sd[p + "mlp.up_proj.weight"]], axis=0),
            down=sd[p + "mlp.down_proj.weight"]))
    return dict(embedding=sd["model.embed_tokens.weight"],
                lm_head=sd.get("lm_head.weight", sd["model.embed_tokens.weight"]),
                final_norm=sd["model.norm.weight"], layers=layers)


@pytest.mark.parametrize("tie", [True, False], ids=["tied", "untied"])
@torch.inference_mode()
def test_dense_logits_match_transformers(tie):
    model, cfg = hf_pair(tie)
    if tie:
        assert model.lm_head.weight is model.model.embed_tokens.weight
    else:
        assert not torch.equal(model.lm_head.weight, model.model.embed_tokens.weight)
    weights = oracle_weights(model)
    for tokens in ([1, 2, 3, 4, 5, 6], [7, 0, 31, 7, 7, 12, 3, 29, 18, 2, 5]):
        expected = model(torch.tensor([tokens]), use_cache=False).logits[0]
        actual = torch.from_numpy(forward_logits(weights, cfg, tokens)).float()
        torch.testing.assert_close(actual, expected, atol=1e-5, rtol=1e-4)


@torch.inference_mode()
def test_prefix_sharing_prompt_matches_transformers():
    # test_hf_parity.py:72-82: a second prompt sharing the first two tokens.
    model, cfg = hf_pair(True)
    weights = oracle_weights(model)
    expected = model(torch.tensor([[1, 2, 7]]), use_cache=False).logits[0, -1]
    actual = torch.from_numpy(forward_logits(weights, cfg, [1, 2, 7])[-1]).float()
    torch.testing.assert_close(actual, expected, atol=1e-5, rtol=1e-4)


@pytest.mark.parametrize("tie", [True, False], ids=["tied", "untied"])
@torch.inference_mode()
def test_greedy_generation_matches_transformers(tie):
    # test_hf_parity.py:93-113: four greedy tokens for each prompt, picked by
    # argmax of the transformers model's last row.
    model, cfg = hf_pair(tie)
    weights = oracle_weights(model)
    for prompt in ([1, 2, 3, 4, 5], [1, 2, 7]):
        ids = torch.tensor([prompt])
        for _ in range(4):
            token = model(ids, use_cache=False).logits[:, -1].argmax(-1, keepdim=True)
            ids = torch.cat((ids, token), dim=-1)
        expected = ids[0, len(prompt):].tolist()
        tokens, gaps = greedy_generate(weights, cfg, prompt, 4)
        assert tokens == expected
        assert min(gaps) > 1e-4  # no near-tie makes this comparison fragile

"""Pins of the dense Qwen3 oracle (oracle/qwen3_dense.py), CPU only.

* The forward equals the same decoder composed from torch's library routines
  (F.rms_norm, F.scaled_dot_product_attention with is_causal, F.silu) in
  float32, to float32 rounding -- a dropped residual, a missing Q/K norm, a
  swapped gate/up half or a wrong GQA head map fails it.
* Appending tokens never changes the logits of earlier positions (causality).
* ``causal_attention`` equals the explicit-loop float64 attention.
* ``greedy_generate`` appends the argmax of the last row each step.
* ``teacher_forced`` on the greedy completion gives back exactly the greedy
  tokens and gaps; on any other completion each choice equals the argmax of
  a separate full forward over the prefix before it; widening the weights
  once (``weights_f64``) and projecting only the last rows change no bit;
  ``token_deficits`` is zero on the greedy path and, for the runner-up
  token, equals the top-2 gap.
"""

from types import SimpleNamespace

import numpy as np
import torch
from torch.nn import functional as F

from oracle.paged_attention import dense_causal_attention_f64
from oracle.qwen3_dense import (causal_attention, forward_logits, greedy_generate,
                                teacher_forced, token_deficits, top2_gap, weights_f64)

CFG = SimpleNamespace(vocab_size=96, hidden_dim=64, norm_eps=1e-6, MLP_inter_dim=96,
                      num_q_head=4, num_kv_head=2, head_dim=16, num_hidden_layer=2,
                      rope_base=10000.0, rope_interleaved=False)


def make_weights(cfg, seed=0):
    rng = np.random.default_rng(seed)

    def normal(*shape, scale=0.2):
        return (scale * rng.standard_normal(shape)).astype(np.float32)

    qkv = (cfg.num_q_head + 2 * cfg.num_kv_head) * cfg.head_dim
    layers = [dict(pre_norm=1 + normal(cfg.hidden_dim, scale=0.1),
                   qkv=normal(qkv, cfg.hidden_dim),
                   q_norm=1 + normal(cfg.head_dim, scale=0.1),
                   k_norm=1 + normal(cfg.head_dim, scale=0.1),
                   out=normal(cfg.hidden_dim, cfg.num_q_head * cfg.head_dim),
                   post_norm=1 + normal(cfg.hidden_dim, scale=0.1),
                   gate_up=normal(2 * cfg.MLP_inter_dim, cfg.hidden_dim),
                   down=normal(cfg.hidden_dim, cfg.MLP_inter_dim))
              for _ in range(cfg.num_hidden_layer)]
    return dict(embedding=normal(cfg.vocab_size, cfg.hidden_dim, scale=1.0),
                lm_head=normal(cfg.vocab_size, cfg.hidden_dim),
                final_norm=1 + normal(cfg.hidden_dim, scale=0.1), layers=layers)


def torch_forward(w, cfg, ids):
    """The decoder from torch.nn.functional routines, float32, CPU."""
    t = torch.from_numpy
    d, eps = cfg.head_dim, cfg.norm_eps
    n = len(ids)
    pos = torch.arange(n, dtype=torch.float32)
    inv = cfg.rope_base ** (-torch.arange(0, d, 2, dtype=torch.float32) / d)
    ang = torch.outer(pos, inv)
    cos, sin = ang.cos()[:, None, :], ang.sin()[:, None, :]

    def rope(x):
        a, b = x[..., :d // 2], x[..., d // 2:]
        return torch.cat((a * cos - b * sin, b * cos + a * sin), -1)

    h = t(w["embedding"])[torch.tensor(ids)]
    res = None
    for L in w["layers"]:
        res = h if res is None else h + res
        x = F.rms_norm(res, (cfg.hidden_dim,), t(L["pre_norm"]), eps)
        q, k, v = F.linear(x, t(L["qkv"])).split(
            [cfg.num_q_head * d, cfg.num_kv_head * d, cfg.num_kv_head * d], -1)
        q = rope(F.rms_norm(q.reshape(n, cfg.num_q_head, d), (d,), t(L["q_norm"]), eps))
        k = rope(F.rms_norm(k.reshape(n, cfg.num_kv_head, d), (d,), t(L["k_norm"]), eps))
        v = v.reshape(n, cfg.num_kv_head, d)
        g = cfg.num_q_head // cfg.num_kv_head
        a = F.scaled_dot_product_attention(
            q.transpose(0, 1), k.repeat_interleave(g, 1).transpose(0, 1).contiguous(),
            v.repeat_interleave(g, 1).transpose(0, 1).contiguous(), is_causal=True)
        h = F.linear(a.transpose(0, 1).reshape(n, -1), t(L["out"]))
        res = h + res
        x = F.rms_norm(res, (cfg.hidden_dim,), t(L["post_norm"]), eps)
        gate, up = F.linear(x, t(L["gate_up"])).chunk(2, -1)
        h = F.linear(F.silu(gate) * up, t(L["down"]))
    x = F.rms_norm(h + res, (cfg.hidden_dim,), t(w["final_norm"]), eps)
    return F.linear(x, t(w["lm_head"])).numpy()


def test_forward_matches_torch_routines():
    w = make_weights(CFG)
    ids = [5, 17, 3, 3, 90, 41, 0, 62, 7, 7, 7, 12]
    got = forward_logits(w, CFG, ids)
    want = torch_forward(w, CFG, ids)
    np.testing.assert_allclose(got, want, rtol=2e-4, atol=2e-4)


def test_forward_is_causal():
    w = make_weights(CFG, seed=1)
    ids = [4, 8, 15, 16, 23, 42]
    short = forward_logits(w, CFG, ids[:3])
    full = forward_logits(w, CFG, ids)
    np.testing.assert_allclose(full[:3], short, rtol=1e-10, atol=1e-10)


def test_attention_matches_the_loop():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((5, 4, 8))
    k = rng.standard_normal((5, 2, 8))
    v = rng.standard_normal((5, 2, 8))
    np.testing.assert_allclose(causal_attention(q, k, v, 0.3),
                               dense_causal_attention_f64(q, k, v, scale=0.3), atol=1e-12)


def test_greedy_generate_appends_last_row_argmax():
    w = make_weights(CFG, seed=3)
    prompt = [1, 2, 3]
    out, gaps = greedy_generate(w, CFG, prompt, 4)
    assert len(out) == 4 and len(gaps) == 4 and all(g >= 0 for g in gaps)
    seq = list(prompt)
    for tok in out:
        assert tok == int(np.argmax(forward_logits(w, CFG, seq)[-1]))
        seq.append(tok)
    cut, _ = greedy_generate(w, CFG, prompt, 4, eos=out[1])
    assert cut == out[:2]


def test_teacher_forced_on_the_greedy_path_is_greedy_generation():
    w = make_weights(CFG, seed=4)
    prompt = [5, 9, 2, 7]
    out, gaps = greedy_generate(w, CFG, prompt, 5)
    picks, tf_gaps = teacher_forced(w, CFG, prompt, out)
    assert picks == out
    np.testing.assert_allclose(tf_gaps, gaps, rtol=0, atol=1e-12)


def test_teacher_forced_checks_every_position_of_another_path():
    w = make_weights(CFG, seed=5)
    prompt = [1, 2, 3]
    completion = [10, 20, 30, 40]  # not the greedy path
    picks, gaps = teacher_forced(w, CFG, prompt, completion)
    assert len(picks) == len(gaps) == len(completion)
    for i in range(len(completion)):
        row = forward_logits(w, CFG, prompt + completion[:i])[-1]
        assert picks[i] == int(np.argmax(row))
        assert gaps[i] == top2_gap(row)
    assert teacher_forced(w, CFG, prompt, []) == ([], [])


def test_wide_weights_and_last_rows_change_nothing():
    w = make_weights(CFG, seed=6)
    ids = [3, 1, 4, 1, 5, 9, 2, 6]
    full = forward_logits(w, CFG, ids)
    wide = forward_logits(weights_f64(w), CFG, ids)
    assert np.array_equal(full, wide)
    assert np.array_equal(forward_logits(w, CFG, ids, last_rows=3), full[-3:])
    assert top2_gap(np.array([1.0, 4.0, 2.5])) == 1.5 and top2_gap(np.array([2.0])) == float("inf")


def test_token_deficits():
    w = make_weights(CFG, seed=7)
    prompt = [2, 7, 1]
    out, gaps = greedy_generate(w, CFG, prompt, 4)
    assert token_deficits(w, CFG, prompt, out) == [0.0] * 4
    row = forward_logits(w, CFG, prompt)[-1]
    runner_up = int(np.argsort(row)[-2])
    # (the products run over different row counts here, so agreement is to
    # float64 rounding, not bitwise)
    np.testing.assert_allclose(token_deficits(w, CFG, prompt, [runner_up]), [gaps[0]],
                               rtol=1e-12)
    worst = int(np.argmin(row))
    np.testing.assert_allclose(token_deficits(w, CFG, prompt, [worst]),
                               [row.max() - row.min()], rtol=1e-12)
    assert token_deficits(w, CFG, prompt, []) == []

"""Dense CPU restatement of the Qwen3 forward and greedy generation
(test infrastructure only).

TEST INFRASTRUCTURE ONLY: imported by ``tests/`` only, never by the product
package.

``forward_logits`` runs the whole token sequence through the decoder with
plain causal attention -- no KV cache, no paging, no chunking, no scheduler
-- following microinfer/model/qwen3.py:44-65 and
microinfer/layer/transformer.py:212-252: pre-norm layers whose RMSNorm also
carries the residual sum (norm.py:26-35), fused QKV, per-head Q/K RMSNorm,
RoPE (rope.py:6-20), GQA causal softmax attention, the output projection,
SwiGLU (transformer.py:90-98), the final norm and the vocabulary projection.
``greedy_generate`` appends ``argmax`` of the last row's logits (runner.py:
240) until ``max_tokens`` or EOS (engine/scheduler.py:232-243), recomputing
the full sequence each time. What the engine adds -- chunked prefill, mixed
steps, prefix-cache reuse, preemption, graph buckets -- must not change these
tokens.

Arithmetic is float32 for the norms and rotations (the oracle's own
``rms_norm`` / ``rotate``) and float64 for the products and attention.

Pins (tests/test_oracle_qwen3_dense.py): the same forward composed from
torch's library routines (F.rms_norm, F.scaled_dot_product_attention with
is_causal and GQA heads repeated, F.silu) on the CPU; causality (appending
tokens never changes earlier rows); and attention against the explicit-loop
``dense_causal_attention_f64``.
"""

from __future__ import annotations

import numpy as np

from oracle.greedy import greedy_argmax
from oracle.qk_norm_rope import rms_norm, rope_tables, rotate


def _norm(x, residual, weight, eps):
    combined = x if residual is None else x + residual
    return rms_norm(combined, weight, eps, "f32").astype(np.float64), combined


def causal_attention(q, k, v, scale):
    """Causal GQA softmax attention: ``q [T, Hq, D]``, ``k, v [T, Hkv, D]``."""
    t, hq, _ = q.shape
    group = hq // k.shape[1]
    k = np.repeat(k, group, axis=1)
    v = np.repeat(v, group, axis=1)
    scores = np.einsum("qhd,khd->hqk", q, k) * scale
    scores = np.where(np.tril(np.ones((t, t), dtype=bool))[None], scores, -np.inf)
    scores = np.exp(scores - scores.max(-1, keepdims=True))
    probs = scores / scores.sum(-1, keepdims=True)
    return np.einsum("hqk,khd->qhd", probs, v)


def weights_f64(weights: dict) -> dict:
    """The same weights with every product matrix widened to float64 once
    (``forward_logits`` then uses them without copying); norm weights stay
    float32, as the float32 norms read them."""
    wide = ("embedding", "lm_head", "qkv", "out", "gate_up", "down")

    def conv(name, a):
        return a.astype(np.float64) if name in wide else a

    out = {k: conv(k, v) for k, v in weights.items() if k != "layers"}
    out["layers"] = [{k: conv(k, v) for k, v in layer.items()} for layer in weights["layers"]]
    return out


def forward_logits(weights: dict, config, token_ids, last_rows: int | None = None) -> np.ndarray:
    """Logits ``[T, vocab]`` (float64) of every position of ``token_ids``.

    ``weights``: numpy arrays ``embedding``, ``lm_head``, ``final_norm`` and
    ``layers`` (a list of dicts ``pre_norm, qkv, q_norm, k_norm, out,
    post_norm, gate_up, down``), shaped as in the product model (float32, or
    float64 from ``weights_f64``). ``last_rows``: project only the last that
    many positions onto the vocabulary (the others are not needed by a
    caller that checks generated tokens).
    """
    c = config
    ids = np.asarray(token_ids, dtype=np.int64)
    t, d = len(ids), c.head_dim
    cos, sin = rope_tables(max(t, 1), d, c.rope_base)
    cos, sin = cos[:t][:, None, :], sin[:t][:, None, :]
    hidden = weights["embedding"][ids].astype(np.float64, copy=False)
    residual = None
    q_w, kv_w = c.num_q_head * d, c.num_kv_head * d
    for layer in weights["layers"]:
        x, residual = _norm(hidden, residual, layer["pre_norm"], c.norm_eps)
        qkv = x @ layer["qkv"].T.astype(np.float64, copy=False)
        q = qkv[:, :q_w].reshape(t, c.num_q_head, d)
        k = qkv[:, q_w:q_w + kv_w].reshape(t, c.num_kv_head, d)
        v = qkv[:, q_w + kv_w:].reshape(t, c.num_kv_head, d)
        q = rotate(rms_norm(q, layer["q_norm"], c.norm_eps, "f32"), cos, sin,
                   interleaved=c.rope_interleaved, dtype="f32").astype(np.float64)
        k = rotate(rms_norm(k, layer["k_norm"], c.norm_eps, "f32"), cos, sin,
                   interleaved=c.rope_interleaved, dtype="f32").astype(np.float64)
        attn = causal_attention(q, k, v, 1.0 / np.sqrt(d))
        hidden = attn.reshape(t, q_w) @ layer["out"].T.astype(np.float64, copy=False)
        x, residual = _norm(hidden, residual, layer["post_norm"], c.norm_eps)
        gate_up = x @ layer["gate_up"].T.astype(np.float64, copy=False)
        gate, up = np.split(gate_up, 2, axis=-1)
        hidden = (gate / (1.0 + np.exp(-gate)) * up) @ layer["down"].T.astype(np.float64, copy=False)
    final, _ = _norm(hidden, residual, weights["final_norm"], c.norm_eps)
    if last_rows is not None:
        final = final[max(0, t - last_rows):]
    return final @ weights["lm_head"].T.astype(np.float64, copy=False)


def top2_gap(row) -> float:
    """Distance between the two largest logits of ``row`` (inf for one logit)."""
    if row.size < 2:
        return float("inf")
    top2 = np.partition(np.asarray(row, dtype=np.float64), row.size - 2)[-2:]
    return float(top2[1] - top2[0])


def teacher_forced(weights: dict, config, prompt, completion):
    """For each token of ``completion``: the oracle's greedy choice and top-2
    gap at that position, given the prompt and the completion's earlier
    tokens (one forward over ``prompt + completion[:-1]``).

    A generator whose tokens all equal these choices is the oracle's greedy
    generation; where they differ only a near-tie (small gap) may have
    flipped, and later positions are still checked, on the generator's own
    path."""
    completion = list(completion)
    if not completion:
        return [], []
    tokens = list(prompt) + completion[:-1]
    rows = forward_logits(weights, config, tokens, last_rows=len(completion))
    picks = [int(t) for t in greedy_argmax(rows)]
    return picks, [top2_gap(r) for r in rows]


def token_deficits(weights: dict, config, prompt, completion) -> list[float]:
    """For each token of ``completion``: how far its logit lies below the
    best logit at that position (0 where it is the oracle's greedy choice),
    given the prompt and the completion's earlier tokens (one forward over
    ``prompt + completion[:-1]``). A generator whose arithmetic differs only
    by rounding keeps every deficit below the logit error that rounding can
    cause."""
    completion = list(completion)
    if not completion:
        return []
    rows = forward_logits(weights, config, list(prompt) + completion[:-1],
                          last_rows=len(completion))
    return [float(row.max() - row[tok]) for row, tok in zip(rows, completion)]


def greedy_generate(weights: dict, config, prompt, max_tokens: int, eos: int | None = None):
    """Greedy completion of ``prompt`` and, per generated token, the gap
    between the two largest logits it was chosen from (near-ties can flip
    under other rounding)."""
    tokens, out, gaps = list(prompt), [], []
    for _ in range(max_tokens):
        row = forward_logits(weights, config, tokens)[-1]
        token = int(greedy_argmax(row[None])[0])
        top2 = np.sort(row)[-2:] if row.size > 1 else np.array([row[0], -np.inf])
        gaps.append(float(top2[1] - top2[0]))
        out.append(token)
        tokens.append(token)
        if eos is not None and token == eos:
            break
    return out, gaps

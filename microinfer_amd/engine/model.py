"""The Qwen3 decoder the engine drives, on the HIP attention path.

Same architecture and forward as ``QwenModel`` / ``TransformerLayer`` /
``Attention`` / ``FFN`` / ``FuseLayerNorm`` (microinfer/model/qwen3.py:8-65,
microinfer/layer/transformer.py:36-252, microinfer/layer/norm.py:20-35):
pre-norm layers whose norms also carry the residual sum, fused QKV and
gate/up projections, per-head Q/K RMSNorm, split-half (or interleaved) RoPE,
GQA attention over the paged KV cache, SwiGLU, a final norm and an untied
(or tied) vocabulary projection; ``compute_logits`` keeps only each request's
last row on prefill (qwen3.py:57-65).

On this path the per-layer Q/K norm + RoPE + KV append is one HIP launch
(``mi_qk_norm_rope_append``), attention is the HIP paged decode / varlen
prefill (``paged_attention_meta`` / ``varlen_attention``), and RMSNorm with
its residual sum and the SwiGLU gate are HIP launches too (``hip_dense``:
the counterparts of the reference's compiled ``_compiled_add_rms_norm`` /
``_compiled_swiglu``), as are the projections of decode batches (up to 64
rows) where the HIP product is measured faster than torch's
(``prefer_hip_linear``); the rest stay on torch (hipBLASLt). Weights are
random:
N(0, 0.02) from a seeded generator, norm weights 1, since no checkpoint is
available to load (``init_std`` sets the spread).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch.nn import functional as F

from microinfer_amd.layer.hip_dense import (hip_linear, hip_linear_swiglu, hip_rms_norm_residual,
                                            hip_silu_mul, prefer_hip_linear, supported_rows)
from microinfer_amd.layer.hip_qk_norm_rope import qk_norm_rope_append, rope_tables
from microinfer_amd.layer.paged_attention import paged_attention_meta, varlen_attention


@dataclass
class QwenConfig:
    """Model dimensions (microinfer/config/config.py:6-20); Qwen3-0.6B defaults."""
    vocab_size: int = 151936
    hidden_dim: int = 1024
    norm_eps: float = 1e-6
    MLP_inter_dim: int = 3072
    num_q_head: int = 16
    num_kv_head: int = 8
    head_dim: int = 128
    num_hidden_layer: int = 28
    max_pos_embed: int = 40960
    rope_base: float = 1000000.0
    rope_interleaved: bool = False
    tie_word_embeddings: bool = False


@dataclass
class _Layer:
    pre_norm: torch.Tensor
    qkv: torch.Tensor  # [(Hq + 2 Hkv) D, H]
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    out: torch.Tensor  # [H, Hq D]
    post_norm: torch.Tensor
    gate_up: torch.Tensor  # [2 I, H]
    down: torch.Tensor  # [H, I]


class Qwen3Model:
    """Weights plus the packed-token forward over a bound KV cache."""

    def __init__(self, config: QwenConfig, *, dtype=torch.bfloat16, device="cuda", seed=0,
                 init_std: float = 0.02, hip_dense: bool = True):
        c = config
        if c.num_q_head % c.num_kv_head or c.head_dim % 2:
            raise ValueError("invalid GQA head ratio or RoPE dimension")
        self.config, self.dtype, self.device = c, dtype, torch.device(device)
        gen = torch.Generator(device=self.device).manual_seed(seed)

        def normal(*shape):
            return (init_std * torch.randn(shape, generator=gen, device=self.device)).to(dtype)

        def ones(n):
            return torch.ones(n, dtype=dtype, device=self.device)

        qkv_rows = (c.num_q_head + 2 * c.num_kv_head) * c.head_dim
        self.embedding = normal(c.vocab_size, c.hidden_dim)
        self.layers = [
            _Layer(ones(c.hidden_dim), normal(qkv_rows, c.hidden_dim), ones(c.head_dim),
                   ones(c.head_dim), normal(c.hidden_dim, c.num_q_head * c.head_dim),
                   ones(c.hidden_dim), normal(2 * c.MLP_inter_dim, c.hidden_dim),
                   normal(c.hidden_dim, c.MLP_inter_dim))
            for _ in range(c.num_hidden_layer)
        ]
        self.final_norm = ones(c.hidden_dim)
        self.lm_head = self.embedding if c.tie_word_embeddings else normal(c.vocab_size,
                                                                           c.hidden_dim)
        self.cos, self.sin = rope_tables(c.max_pos_embed, c.head_dim, c.rope_base,
                                         device=self.device)
        self.caches = None
        self.hip_dense = hip_dense and dtype in (torch.bfloat16, torch.float16)

    def bind_caches(self, caches) -> None:
        """One ``LayerKVCache`` per layer (``[N, B, Hkv, D]`` views)."""
        if len(caches) != len(self.layers):
            raise ValueError("one cache per layer is required")
        self.caches = list(caches)

    def _norm(self, x, residual, weight):
        if self.hip_dense and supported_rows(x, residual):
            return hip_rms_norm_residual(x, residual, weight, self.config.norm_eps)
        combined = x if residual is None else x + residual
        return F.rms_norm(combined, (combined.shape[-1],), weight, self.config.norm_eps), combined

    def _linear(self, x, weight):
        if self.hip_dense and prefer_hip_linear(x, weight):
            return hip_linear(x, weight)
        return F.linear(x, weight)

    def _swiglu(self, gate_up):
        if self.hip_dense and supported_rows(gate_up):
            return hip_silu_mul(gate_up)
        gate, up = gate_up.chunk(2, dim=-1)
        return F.silu(gate) * up

    def _ffn_gate(self, x, gate_up):
        """SwiGLU of the gate/up projection: one fused launch where the HIP
        projection is preferred, else the projection and then the gate."""
        if self.hip_dense and prefer_hip_linear(x, gate_up) and gate_up.shape[0] % 32 == 0:
            return hip_linear_swiglu(x, gate_up)
        return self._swiglu(self._linear(x, gate_up))

    def forward(self, input_ids, positions, metadata):
        """Hidden states ``[T, H]`` of the packed tokens of one step."""
        c = self.config
        if self.caches is None:
            raise RuntimeError("bind the KV caches before running the model")
        tokens = input_ids.shape[0]
        q_width, kv_width = c.num_q_head * c.head_dim, c.num_kv_head * c.head_dim
        direct = metadata.is_prefill and metadata.direct_prefill
        hidden, residual = F.embedding(input_ids, self.embedding), None
        for layer, cache in zip(self.layers, self.caches):
            x, residual = self._norm(hidden, residual, layer.pre_norm)
            qkv = self._linear(x, layer.qkv)
            rotated = qk_norm_rope_append(
                qkv, q_weight=layer.q_norm, k_weight=layer.k_norm, eps=c.norm_eps,
                cos_table=self.cos, sin_table=self.sin, positions=positions,
                num_q_heads=c.num_q_head, num_kv_heads=c.num_kv_head, head_dim=c.head_dim,
                interleaved=c.rope_interleaved, slot_mapping=metadata.slot_mapping,
                key_cache=cache.keys, value_cache=cache.values, return_k=direct)
            if direct:  # no cached prefix: attend over this step's own K/V
                q, k = rotated
                v = qkv[:, q_width + kv_width:].reshape(tokens, c.num_kv_head, c.head_dim)
                attn = varlen_attention(q, k, v.contiguous(), metadata)
            else:
                attn = paged_attention_meta(rotated, cache.keys, cache.values, metadata)
            hidden = self._linear(attn.reshape(tokens, q_width), layer.out)
            x, residual = self._norm(hidden, residual, layer.post_norm)
            hidden = self._linear(self._ffn_gate(x, layer.gate_up), layer.down)
        return self._norm(hidden, residual, self.final_norm)[0]

    def compute_logits(self, hidden, metadata):
        """Vocabulary logits of each request's last row (prefill) or every
        row (decode)."""
        if metadata.is_prefill and metadata.cu_seqlens_q is not None:
            hidden = hidden[metadata.cu_seqlens_q[1:].long() - 1]
        return self._linear(hidden, self.lm_head)

    def host_weights(self) -> dict:
        """float32 numpy copies of every weight, keyed as the dense oracle
        reads them."""
        def arr(t):
            return t.float().cpu().numpy()

        names = ("pre_norm", "qkv", "q_norm", "k_norm", "out", "post_norm", "gate_up", "down")
        return dict(embedding=arr(self.embedding), lm_head=arr(self.lm_head),
                    final_norm=arr(self.final_norm),
                    layers=[{n: arr(getattr(layer, n)) for n in names} for layer in self.layers])

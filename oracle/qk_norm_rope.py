"""numpy restatement of the attention block's Q/K RMSNorm + RoPE + KV append.

Test infrastructure: only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s cpu_baseline leg may import this module. It is what results are
compared with, never the thing measured or shipped.

Follows, for one layer's fused QKV rows ``[T, (Hq + 2 Hkv) * D]``:

* ``rms_norm`` -- ``F.rms_norm`` over the head dimension with the norm weight,
  as ``Attention.q_norm`` / ``k_norm`` apply it (microinfer/layer/norm.py:26-35,
  microinfer/layer/transformer.py:119-124, :229-230): computed in float32,
  ``x * (1 / sqrt(mean(x^2) + eps)) * w``, rounded once to the input dtype.
* ``rope_tables`` -- ``RotaryCache.ensure`` (microinfer/layer/rope.py:45-55):
  ``inv = base ** (-arange(0, D, 2) / D)``, ``angles = outer(arange(L), inv)``,
  float32 cos and sin.
* ``rotate`` -- ``_rotate`` (microinfer/layer/rope.py:6-20): float32
  split-half (Qwen) or interleaved rotation by the position's angles, rounded
  to the input dtype.
* ``qk_norm_rope_append`` -- ``Attention.forward``'s Q/K path
  (transformer.py:186-233: split the fused QKV, norm, rotate) followed by the
  append that ``CachedAttention.forward`` does first (cached_attention.py:
  76-85, kv_cache.py:52-79): K (normalised, rotated) and V (as projected) go to
  ``slot_mapping``; slot -1 is skipped.

Pinned by tests/test_oracle_qk_norm_rope.py: ``rms_norm`` against
``torch.nn.functional.rms_norm`` (a library routine) in float32 and bfloat16;
RoPE by its defining properties -- position 0 is the identity, every rotated
pair keeps its length, ``<rope(q, m), rope(k, n)>`` depends only on ``m - n``,
interleaved equals split-half under the even/odd permutation -- and the
tables by the closed form ``angle(p, i) = p * base^(-2i/D)`` in float64; the
append by ``kv_append``'s own pins (oracle/paged_attention.py).
"""

from __future__ import annotations

import numpy as np

from oracle.numerics import round_to_dtype
from oracle.paged_attention import kv_append


def rms_norm(x, weight, eps: float, dtype: str) -> np.ndarray:
    """RMSNorm over the last axis in float32, one rounding to ``dtype``."""
    x = np.asarray(x, dtype=np.float32)
    w = np.asarray(weight, dtype=np.float32)
    mean_sq = np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32)
    inv = np.float32(1.0) / np.sqrt(mean_sq + np.float32(eps), dtype=np.float32)
    return round_to_dtype(x * inv * w, dtype)


def rope_tables(max_len: int, dim: int, base: float):
    """float32 cos and sin tables ``[max_len, dim / 2]``."""
    if max_len <= 0 or dim <= 0 or dim % 2 or base <= 0:
        raise ValueError("invalid RoPE cache dimensions/base")
    exponent = -np.arange(0, dim, 2, dtype=np.float32) / np.float32(dim)
    inv = np.power(np.float32(base), exponent, dtype=np.float32)
    angles = np.outer(np.arange(max_len, dtype=np.float32), inv).astype(np.float32)
    return np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32)


def rotate(x, cosine, sine, *, interleaved: bool, dtype: str) -> np.ndarray:
    """Rotate the last axis by (cosine, sine) (broadcast over heads)."""
    x = np.asarray(x, dtype=np.float32)
    cosine = np.asarray(cosine, dtype=np.float32)
    sine = np.asarray(sine, dtype=np.float32)
    if interleaved:
        first, second = x[..., 0::2], x[..., 1::2]
        out = np.stack((first * cosine - second * sine, first * sine + second * cosine), -1)
        out = out.reshape(x.shape)
    else:
        half = x.shape[-1] // 2
        first, second = x[..., :half], x[..., half:]
        out = np.concatenate((first * cosine - second * sine, second * cosine + first * sine), -1)
    return round_to_dtype(out, dtype)


def qk_norm_rope_append(qkv, q_weight, k_weight, eps: float, cos_table, sin_table, positions,
                        slot_mapping, key_cache, value_cache, *, num_q_heads: int,
                        num_kv_heads: int, head_dim: int, interleaved: bool, dtype: str):
    """Returns (q, k) after norm + RoPE; writes K and V rows into the caches.

    ``qkv`` holds the fused projection rows (values of ``dtype`` as float32),
    ``key_cache`` / ``value_cache`` are ``[N, B, Hkv, D]`` float32 arrays
    updated in place.
    """
    qkv = np.asarray(qkv, dtype=np.float32)
    t = qkv.shape[0]
    hq, hkv, d = num_q_heads, num_kv_heads, head_dim
    q = qkv[:, : hq * d].reshape(t, hq, d)
    k = qkv[:, hq * d : (hq + hkv) * d].reshape(t, hkv, d)
    v = qkv[:, (hq + hkv) * d : (hq + 2 * hkv) * d].reshape(t, hkv, d)
    index = np.asarray(positions, dtype=np.int64)
    cosine = np.asarray(cos_table, dtype=np.float32)[index][:, None, :]
    sine = np.asarray(sin_table, dtype=np.float32)[index][:, None, :]
    q_out = rotate(rms_norm(q, q_weight, eps, dtype), cosine, sine,
                   interleaved=interleaved, dtype=dtype)
    k_out = rotate(rms_norm(k, k_weight, eps, dtype), cosine, sine,
                   interleaved=interleaved, dtype=dtype)
    kv_append(key_cache, value_cache, slot_mapping, k_out, v)
    return q_out, k_out

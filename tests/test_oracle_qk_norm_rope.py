"""Pins of the Q/K RMSNorm + RoPE + append oracle (oracle/qk_norm_rope.py), CPU only.

* rms_norm against torch.nn.functional.rms_norm (a library routine), float32
  to 1e-6 and bfloat16 to one bf16 ulp.
* rope_tables against the closed form angle(p, i) = p * base^(-2i/D) in
  float64.
* rotate by RoPE's defining properties, each chosen so a plausible slip fails
  one of them: position 0 is the identity; every rotated pair keeps its
  length (a dropped or doubled term breaks it); a unit vector in the first
  half lands at (cos, sin) (a flipped sign or swapped half breaks it);
  <rope(q, m), rope(k, n)> depends only on m - n; interleaved equals
  split-half under the even/odd permutation.
* qk_norm_rope_append composes the two and appends through kv_append (whose
  own pins are in test_oracle_paged_attention.py): the cache rows at the
  slots equal the returned K rows and the raw V rows, slot -1 is skipped.
"""

import numpy as np
import pytest
import torch

from oracle.numerics import bf16_bits_to_f32, f32_to_bf16_bits
from oracle.qk_norm_rope import qk_norm_rope_append, rms_norm, rope_tables, rotate


def _bf16(x):
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(x, dtype=np.float32)))


def test_rms_norm_matches_torch_f32():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((7, 5, 128)).astype(np.float32) * 3
    w = rng.standard_normal(128).astype(np.float32)
    want = torch.nn.functional.rms_norm(torch.from_numpy(x), (128,), torch.from_numpy(w), 1e-6)
    np.testing.assert_allclose(rms_norm(x, w, 1e-6, "f32"), want.numpy(), rtol=1e-5, atol=1e-6)


def test_rms_norm_matches_torch_bf16_within_one_ulp():
    rng = np.random.default_rng(1)
    x = _bf16(rng.standard_normal((64, 128)) * 2)
    w = _bf16(1 + 0.1 * rng.standard_normal(128))
    want = torch.nn.functional.rms_norm(
        torch.from_numpy(x).to(torch.bfloat16), (128,), torch.from_numpy(w).to(torch.bfloat16),
        1e-6).float().numpy()
    got = rms_norm(x, w, 1e-6, "bf16")
    ulp = np.abs(f32_to_bf16_bits(got).astype(np.int32) - f32_to_bf16_bits(want).astype(np.int32))
    assert ulp.max() <= 1
    assert (ulp == 0).mean() > 0.95


def test_rms_norm_unit_weight_gives_unit_rms_and_eps_matters():
    x = np.full((1, 64), 3.0, dtype=np.float32)
    y = rms_norm(x, np.ones(64, dtype=np.float32), 0.0, "f32")
    np.testing.assert_allclose(y, np.ones_like(y), rtol=1e-6)
    # eps enters under the root: x = 0 stays 0, a tiny x is damped.
    assert np.all(rms_norm(np.zeros((1, 64)), np.ones(64), 1e-6, "f32") == 0)
    small = rms_norm(np.full((1, 64), 1e-4), np.ones(64), 1e-6, "f32")
    np.testing.assert_allclose(small, 1e-4 / np.sqrt(1e-8 + 1e-6), rtol=1e-5)


def test_rope_tables_closed_form():
    cos, sin = rope_tables(64, 128, 1_000_000.0)
    p = np.arange(64)[:, None].astype(np.float64)
    i = np.arange(64)[None, :].astype(np.float64)
    angle = p * 1_000_000.0 ** (-2 * i / 128)
    np.testing.assert_allclose(cos, np.cos(angle), atol=5e-6)
    np.testing.assert_allclose(sin, np.sin(angle), atol=5e-6)
    assert np.all(cos[0] == 1) and np.all(sin[0] == 0)
    with pytest.raises(ValueError):
        rope_tables(8, 7, 10000.0)


@pytest.mark.parametrize("interleaved", [False, True])
def test_rotation_identity_and_pair_lengths(interleaved):
    rng = np.random.default_rng(2)
    cos, sin = rope_tables(512, 128, 10000.0)
    x = rng.standard_normal((5, 3, 128)).astype(np.float32)
    pos = np.array([0, 1, 17, 300, 511])
    out = rotate(x, cos[pos][:, None], sin[pos][:, None], interleaved=interleaved, dtype="f32")
    assert np.array_equal(out[0], x[0])  # cos 1, sin 0
    if interleaved:
        pairs_in = x[..., 0::2] ** 2 + x[..., 1::2] ** 2
        pairs_out = out[..., 0::2] ** 2 + out[..., 1::2] ** 2
    else:
        pairs_in = x[..., :64] ** 2 + x[..., 64:] ** 2
        pairs_out = out[..., :64] ** 2 + out[..., 64:] ** 2
    np.testing.assert_allclose(pairs_out, pairs_in, rtol=1e-5, atol=1e-6)


def test_rotation_direction_on_unit_vectors():
    cos, sin = rope_tables(100, 8, 10000.0)
    for i in range(4):
        e = np.zeros(8, dtype=np.float32)
        e[i] = 1
        out = rotate(e[None], cos[37][None], sin[37][None], interleaved=False, dtype="f32")[0]
        expect = np.zeros(8, dtype=np.float32)
        expect[i], expect[i + 4] = cos[37, i], sin[37, i]
        np.testing.assert_allclose(out, expect, atol=1e-7)
        e2 = np.zeros(8, dtype=np.float32)
        e2[2 * i] = 1
        out2 = rotate(e2[None], cos[37][None], sin[37][None], interleaved=True, dtype="f32")[0]
        expect2 = np.zeros(8, dtype=np.float32)
        expect2[2 * i], expect2[2 * i + 1] = cos[37, i], sin[37, i]
        np.testing.assert_allclose(out2, expect2, atol=1e-7)


@pytest.mark.parametrize("interleaved", [False, True])
def test_scores_depend_only_on_relative_position(interleaved):
    rng = np.random.default_rng(3)
    cos, sin = rope_tables(4096, 64, 10000.0)
    q = rng.standard_normal(64).astype(np.float32)
    k = rng.standard_normal(64).astype(np.float32)

    def score(m, n):
        qm = rotate(q[None], cos[m][None], sin[m][None], interleaved=interleaved, dtype="f32")[0]
        kn = rotate(k[None], cos[n][None], sin[n][None], interleaved=interleaved, dtype="f32")[0]
        return float(np.dot(qm.astype(np.float64), kn.astype(np.float64)))

    base = score(10, 3)
    for shift in (1, 50, 700):
        assert abs(score(10 + shift, 3 + shift) - base) <= 2e-3 * (1 + abs(base))
    assert abs(score(10, 4) - base) > 1e-3  # a different offset gives another score


def test_interleaved_is_split_half_under_even_odd_permutation():
    rng = np.random.default_rng(4)
    cos, sin = rope_tables(64, 128, 10000.0)
    x = rng.standard_normal((6, 128)).astype(np.float32)
    pos = rng.integers(0, 64, 6)
    perm = np.concatenate([np.arange(0, 128, 2), np.arange(1, 128, 2)])
    inter = rotate(x, cos[pos], sin[pos], interleaved=True, dtype="f32")
    split = rotate(x[:, perm], cos[pos], sin[pos], interleaved=False, dtype="f32")
    np.testing.assert_array_equal(inter[:, perm], split)


def test_append_composition_and_skips():
    rng = np.random.default_rng(5)
    hq, hkv, d, bs = 4, 2, 16, 4
    t = 5
    qkv = _bf16(rng.standard_normal((t, (hq + 2 * hkv) * d)))
    qw = _bf16(1 + 0.1 * rng.standard_normal(d))
    kw = _bf16(1 + 0.1 * rng.standard_normal(d))
    cos, sin = rope_tables(64, d, 10000.0)
    pos = np.array([0, 5, 9, 63, 2])
    slots = np.array([3, -1, 8, 0, 13])
    kc = np.zeros((4, bs, hkv, d), dtype=np.float32)
    vc = np.zeros_like(kc)
    q, k = qk_norm_rope_append(qkv, qw, kw, 1e-6, cos, sin, pos, slots, kc, vc,
                               num_q_heads=hq, num_kv_heads=hkv, head_dim=d,
                               interleaved=False, dtype="bf16")
    q_raw = qkv[:, : hq * d].reshape(t, hq, d)
    np.testing.assert_array_equal(
        q, rotate(rms_norm(q_raw, qw, 1e-6, "bf16"), cos[pos][:, None], sin[pos][:, None],
                  interleaved=False, dtype="bf16"))
    v_raw = qkv[:, (hq + hkv) * d:].reshape(t, hkv, d)
    for i, s in enumerate(slots):
        if s < 0:
            continue
        np.testing.assert_array_equal(kc[s // bs, s % bs], k[i])
        np.testing.assert_array_equal(vc[s // bs, s % bs], v_raw[i])
    written = {(s // bs, s % bs) for s in slots if s >= 0}
    for b in range(4):
        for o in range(bs):
            if (b, o) not in written:
                assert not kc[b, o].any() and not vc[b, o].any()

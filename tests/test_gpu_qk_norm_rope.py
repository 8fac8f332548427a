"""Fused Q/K RMSNorm + RoPE + KV append (mi_qk_norm_rope_append) against the oracle.

The oracle (oracle/qk_norm_rope.py) restates Attention.forward's norm and
rotation (microinfer/layer/transformer.py:186-233, norm.py:26-35,
rope.py:6-20) and the append (cached_attention.py:76-85). Tolerances: float32
within 1e-5 relative; 16-bit results within two units in the last place of
the element type (the kernel's float32 sum of squares runs in another order
than numpy's, which can move a rounding of the normalised value by one ulp
and the rotated value by up to two) with at least 90 % of the elements bit
for bit equal. V rows are copied bit for bit; K in the cache equals the K the
call returns, bit for bit. The cases: both rotation layouts, the 0.6B and 8B
head shapes, head dims 64/128/256, strided fused rows, int32 and int64
positions, slot -1 and out-of-range positions, poison outside the written
slots, no-append mode, and hipGraph replay with new positions and slots.
"""

import numpy as np
import pytest
import torch

from microinfer_amd.layer.hip_qk_norm_rope import qk_norm_rope_append
from microinfer_amd.runner import capture_graph
from oracle import qk_norm_rope as ref
from tests.support import as_f32

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAMES = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}


def _case(tokens, hq, hkv, d, dtype, seed, *, table_len=4096, extra_width=0):
    gen = torch.Generator().manual_seed(seed)
    width = (hq + 2 * hkv) * d
    qkv_full = torch.randn(tokens, width + extra_width, generator=gen) * 2
    qkv = qkv_full.to(dtype).to(DEV)[:, :width] if extra_width else qkv_full.to(dtype).to(DEV)
    qw = (1 + 0.2 * torch.randn(d, generator=gen)).to(dtype).to(DEV)
    kw = (1 + 0.2 * torch.randn(d, generator=gen)).to(dtype).to(DEV)
    cos, sin = ref.rope_tables(table_len, d, 1_000_000.0)
    return qkv, qw, kw, torch.from_numpy(cos).to(DEV), torch.from_numpy(sin).to(DEV)


def _close(got, want, dtype):
    got, want = as_f32(got), np.asarray(want, dtype=np.float32)
    if dtype == torch.float32:
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)
        return
    # Two units in the last place of the 16-bit type, relative to the value or
    # to 1 (normalised rows are O(1); a rotated value near zero comes from
    # cancelling O(1) terms, so its error is on the scale of those terms).
    rel = 2.0 ** (-6 if dtype == torch.bfloat16 else -9)
    err = np.abs(got - want)
    assert np.all(err <= rel * np.maximum(np.abs(want), 1.0)), float(err.max())
    assert np.mean(got == want) >= 0.9


def _oracle(qkv, qw, kw, cos, sin, pos, slots, kc, vc, hq, hkv, d, interleaved, dtype):
    kc_h, vc_h = as_f32(kc), as_f32(vc)
    q, k = ref.qk_norm_rope_append(
        as_f32(qkv), as_f32(qw), as_f32(kw), 1e-6, cos.cpu().numpy(), sin.cpu().numpy(),
        pos.cpu().numpy(), slots.cpu().numpy(), kc_h, vc_h, num_q_heads=hq,
        num_kv_heads=hkv, head_dim=d, interleaved=interleaved, dtype=NAMES[dtype])
    return q, k, kc_h, vc_h


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("interleaved", [False, True])
@pytest.mark.parametrize("hq,hkv", [(16, 8), (32, 8)])
def test_matches_oracle_with_append(dtype, interleaved, hq, hkv):
    d, bs, blocks, tokens = 128, 16, 64, 37
    qkv, qw, kw, cos, sin = _case(tokens, hq, hkv, d, dtype, seed=hq + int(interleaved))
    gen = torch.Generator().manual_seed(9)
    pos = torch.randint(0, 4096, (tokens,), generator=gen).to(DEV)
    slots = torch.randperm(blocks * bs, generator=gen)[:tokens].to(torch.int32)
    slots[3] = -1
    slots = slots.to(DEV)
    kc = torch.full((blocks, bs, hkv, d), 7.0, dtype=dtype, device=DEV)  # poison
    vc = torch.full_like(kc, -7.0)
    q_want, k_want, kc_want, vc_want = _oracle(qkv, qw, kw, cos, sin, pos, slots, kc, vc,
                                               hq, hkv, d, interleaved, dtype)
    q, k = qk_norm_rope_append(qkv, q_weight=qw, k_weight=kw, eps=1e-6, cos_table=cos,
                               sin_table=sin, positions=pos, num_q_heads=hq,
                               num_kv_heads=hkv, head_dim=d, interleaved=interleaved,
                               slot_mapping=slots, key_cache=kc, value_cache=vc,
                               return_k=True)
    _close(q, q_want, dtype)
    _close(k, k_want, dtype)
    # Cache rows: K equals the returned K, V the projected V, bit for bit; the
    # poison everywhere else is untouched.
    s = slots.cpu().numpy()
    v_raw = qkv[:, (hq + hkv) * d:].reshape(tokens, hkv, d)
    touched = torch.zeros(blocks, bs, dtype=torch.bool)
    for i, slot in enumerate(s):
        if slot < 0:
            continue
        b, o = divmod(int(slot), bs)
        touched[b, o] = True
        assert torch.equal(kc[b, o], k[i])
        assert torch.equal(vc[b, o], v_raw[i])
    keep = ~touched.to(DEV)
    assert bool((kc[keep] == 7.0).all()) and bool((vc[keep] == -7.0).all())
    _close(kc, kc_want, dtype)
    assert np.array_equal(as_f32(vc), vc_want)


@pytest.mark.parametrize("d", [64, 256])
@pytest.mark.parametrize("interleaved", [False, True])
def test_head_dims(d, interleaved):
    hq, hkv, tokens = 8, 2, 9
    dtype = torch.bfloat16
    qkv, qw, kw, cos, sin = _case(tokens, hq, hkv, d, dtype, seed=d)
    pos = torch.arange(tokens, device=DEV) * 97
    q, k = qk_norm_rope_append(qkv, q_weight=qw, k_weight=kw, eps=1e-6, cos_table=cos,
                               sin_table=sin, positions=pos, num_q_heads=hq,
                               num_kv_heads=hkv, head_dim=d, interleaved=interleaved,
                               return_k=True)
    kc = np.zeros((4, 16, hkv, d), dtype=np.float32)
    q_want, k_want = ref.qk_norm_rope_append(
        as_f32(qkv), as_f32(qw), as_f32(kw), 1e-6, cos.cpu().numpy(), sin.cpu().numpy(),
        pos.cpu().numpy(), np.full(tokens, -1), kc, kc.copy(), num_q_heads=hq,
        num_kv_heads=hkv, head_dim=d, interleaved=interleaved, dtype="bf16")
    _close(q, q_want, dtype)
    _close(k, k_want, dtype)


@pytest.mark.parametrize("pos_dtype", [torch.int32, torch.int64])
def test_strided_rows_positions_and_out_of_range(pos_dtype):
    hq, hkv, d, bs, tokens = 16, 8, 128, 16, 12
    dtype = torch.bfloat16
    qkv, qw, kw, cos, sin = _case(tokens, hq, hkv, d, dtype, seed=5, table_len=512,
                                  extra_width=3 * d)
    assert qkv.stride(0) > qkv.shape[1]
    pos = torch.tensor([0, 1, 511, 512, -1, 100, 7, 3, 300, 2, 9, 400], dtype=pos_dtype,
                       device=DEV)
    slots = torch.arange(tokens, dtype=torch.int32, device=DEV) + 16
    kc = torch.full((4, bs, hkv, d), 3.0, dtype=dtype, device=DEV)
    vc = torch.full_like(kc, 3.0)
    q, k = qk_norm_rope_append(qkv, q_weight=qw, k_weight=kw, eps=1e-6, cos_table=cos,
                               sin_table=sin, positions=pos, num_q_heads=hq,
                               num_kv_heads=hkv, head_dim=d, slot_mapping=slots,
                               key_cache=kc, value_cache=vc, return_k=True)
    bad = [3, 4]  # positions 512 (past the table) and -1
    good = [i for i in range(tokens) if i not in bad]
    assert not q[bad].any() and not k[bad].any()
    for i in bad:  # no append
        b, o = divmod(16 + i, bs)
        assert bool((kc[b, o] == 3.0).all()) and bool((vc[b, o] == 3.0).all())
    kc_h = np.zeros((4, bs, hkv, d), dtype=np.float32)
    q_want, k_want = ref.qk_norm_rope_append(
        as_f32(qkv[good]), as_f32(qw), as_f32(kw), 1e-6, cos.cpu().numpy(), sin.cpu().numpy(),
        pos[good].cpu().numpy(), np.full(len(good), -1), kc_h, kc_h.copy(), num_q_heads=hq,
        num_kv_heads=hkv, head_dim=d, interleaved=False, dtype="bf16")
    _close(q[good], q_want, dtype)
    _close(k[good], k_want, dtype)


def test_no_append_leaves_caches_alone_and_errors():
    hq, hkv, d = 16, 8, 128
    qkv, qw, kw, cos, sin = _case(4, hq, hkv, d, torch.bfloat16, seed=6)
    pos = torch.arange(4, device=DEV)
    q = qk_norm_rope_append(qkv, q_weight=qw, k_weight=kw, eps=1e-6, cos_table=cos,
                            sin_table=sin, positions=pos, num_q_heads=hq, num_kv_heads=hkv,
                            head_dim=d)
    assert q.shape == (4, hq, d)
    with pytest.raises(ValueError, match="head_dim"):
        qk_norm_rope_append(qkv, q_weight=qw, k_weight=kw, eps=1e-6, cos_table=cos,
                            sin_table=sin, positions=pos, num_q_heads=hq, num_kv_heads=hkv,
                            head_dim=127)
    with pytest.raises(ValueError, match="both caches"):
        qk_norm_rope_append(qkv, q_weight=qw, k_weight=kw, eps=1e-6, cos_table=cos,
                            sin_table=sin, positions=pos, num_q_heads=hq, num_kv_heads=hkv,
                            head_dim=d, slot_mapping=pos.to(torch.int32))
    with pytest.raises(ValueError, match="float32"):
        qk_norm_rope_append(qkv, q_weight=qw, k_weight=kw, eps=1e-6, cos_table=cos.double(),
                            sin_table=sin, positions=pos, num_q_heads=hq, num_kv_heads=hkv,
                            head_dim=d)
    empty = qk_norm_rope_append(qkv[:0], q_weight=qw, k_weight=kw, eps=1e-6, cos_table=cos,
                                sin_table=sin, positions=pos[:0], num_q_heads=hq,
                                num_kv_heads=hkv, head_dim=d)
    assert empty.shape == (0, hq, d)


def test_graph_replay_with_new_positions_and_slots():
    hq, hkv, d, bs, tokens = 16, 8, 128, 16, 32
    dtype = torch.bfloat16
    qkv, qw, kw, cos, sin = _case(tokens, hq, hkv, d, dtype, seed=7)
    pos = torch.zeros(tokens, dtype=torch.int64, device=DEV)
    slots = torch.zeros(tokens, dtype=torch.int32, device=DEV)
    kc = torch.zeros((64, bs, hkv, d), dtype=dtype, device=DEV)
    vc = torch.zeros_like(kc)
    out = torch.empty((tokens, hq, d), dtype=dtype, device=DEV)

    def step(k_cache, v_cache):
        return qk_norm_rope_append(qkv, q_weight=qw, k_weight=kw, eps=1e-6, cos_table=cos,
                                   sin_table=sin, positions=pos, num_q_heads=hq,
                                   num_kv_heads=hkv, head_dim=d, slot_mapping=slots,
                                   key_cache=k_cache, value_cache=v_cache)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(kc, vc)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with capture_graph(graph):
        out.copy_(step(kc, vc))
    kc_e, vc_e = kc.clone(), vc.clone()  # after the warm-up's writes
    gen = torch.Generator().manual_seed(11)
    for rep in range(3):
        pos.copy_(torch.randint(0, 4096, (tokens,), generator=gen))
        slots.copy_(torch.randperm(64 * bs, generator=gen)[:tokens].to(torch.int32))
        qkv.normal_()
        graph.replay()
        torch.cuda.synchronize()
        eager = step(kc_e, vc_e)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep}"
        assert torch.equal(kc, kc_e) and torch.equal(vc, vc_e), f"replay {rep} caches"

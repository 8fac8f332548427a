"""Host side of the fused Q/K norm + RoPE + append (no GPU).

CPU tensors raise RuntimeError (the product has no CPU fallback), and the C
entry rejects bad sizes and missing pointers with a status and a message
before launching anything.
"""

import pytest
import torch

from microinfer_amd import _lib
from microinfer_amd.layer.hip_qk_norm_rope import qk_norm_rope_append


def test_cpu_tensors_raise_runtime_error():
    qkv = torch.zeros(2, 4 * 8, dtype=torch.bfloat16)
    w = torch.ones(8, dtype=torch.bfloat16)
    table = torch.ones(16, 4)
    with pytest.raises(RuntimeError, match="HIP device only"):
        qk_norm_rope_append(qkv, q_weight=w, k_weight=w, eps=1e-6, cos_table=table,
                            sin_table=table, positions=torch.zeros(2, dtype=torch.int64),
                            num_q_heads=2, num_kv_heads=1, head_dim=8)


def _call(lib, **over):
    args = dict(qkv=1024, ts=64, qw=1024, kw=1024, eps=1e-6, cos=1024, sin=1024, tlen=16,
                pos=1024, pos64=1, slots=None, q=1024, q_ts=32, q_hs=16, k=None, k_ts=0,
                k_hs=0, kc=None, vc=None, c_bs=0, c_ts=0, c_hs=0, tokens=2, hq=2, hkv=1, d=16,
                il=0, bs=0, nb=0, dtype=2)
    args.update(over)
    return lib.mi_qk_norm_rope_append(*args.values(), None)


def test_c_entry_validates_before_launch():
    lib = _lib.load()
    assert _call(lib, d=7) == 2 and "head_dim" in _lib.last_error()
    assert _call(lib, d=8) == 2  # less than two 16-byte bf16 vectors
    assert _call(lib, d=24) == 2 and _call(lib, d=512) == 2
    assert _call(lib, tokens=-1) == 1
    assert _call(lib, qkv=None) == 1 and "null" in _lib.last_error()
    assert _call(lib, ts=32) == 1 and "stride" in _lib.last_error()
    assert _call(lib, qkv=1032) == 1 and "aligned" in _lib.last_error()
    assert _call(lib, cos=1028) == 1 and "aligned" in _lib.last_error()
    assert _call(lib, q_hs=20) == 1 and "aligned" in _lib.last_error()
    assert _call(lib, slots=1024) == 1 and "caches" in _lib.last_error()
    assert _call(lib, slots=1024, kc=1024, vc=1024) == 1 and "cache sizes" in _lib.last_error()
    assert _call(lib, dtype=9) == 1
    assert _call(lib, tokens=0) == 0  # nothing to do


def test_product_rope_tables_match_the_oracle():
    from microinfer_amd.layer.hip_qk_norm_rope import rope_tables
    from oracle.qk_norm_rope import rope_tables as oracle_tables

    cos, sin = rope_tables(2048, 128, 1_000_000.0, device="cpu")
    want_cos, want_sin = oracle_tables(2048, 128, 1_000_000.0)
    assert cos.dtype == torch.float32 and cos.shape == (2048, 64)
    # Both are float32 computations of the same formula; a last-bit difference
    # in a frequency grows with the position: allow 1e-6 + p * 2^-21.
    tol = 1e-6 + torch.arange(2048, dtype=torch.float32)[:, None] * 2.0 ** -21
    assert bool(((cos - torch.from_numpy(want_cos)).abs() <= tol).all())
    assert bool(((sin - torch.from_numpy(want_sin)).abs() <= tol).all())
    assert bool((cos[:16] - torch.from_numpy(want_cos[:16])).abs().max() <= 1e-6)
    with pytest.raises(ValueError):
        rope_tables(16, 7, 10000.0, device="cpu")

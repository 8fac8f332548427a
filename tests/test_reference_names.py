"""The reference-named entry points on the CPU (no kernel launches).

``microinfer_amd.layer.triton_paged_attention`` exports what the reference's
module does (microinfer/layer/triton_paged_attention.py): ``HAS_TRITON``,
``triton_paged_decode``, ``triton_paged_prefill``, ``DEFAULT_SPLIT_K``,
``MIN_PROGRAMS`` and ``_select_split_k``; ``microinfer_amd.layer.
paged_attention`` exports ``_gather_paged_kv`` (paged_attention.py:76). Their
contract violations raise ValueError before anything reaches the device, in
the reference's order (triton_paged_attention.py:276-302, :370-399).
"""

import inspect

import pytest
import torch

from microinfer_amd.layer import paged_attention, triton_paged_attention as tpa
from microinfer_amd.layer.hip_paged_attention import hip_paged_decode, hip_paged_prefill


def test_exports_and_signatures():
    assert tpa.HAS_TRITON is True  # the library loads (no device needed)
    assert paged_attention._gather_paged_kv is paged_attention.gather_paged_kv
    decode = inspect.signature(tpa.triton_paged_decode)
    assert list(decode.parameters) == ["query", "key_cache", "value_cache", "block_tables",
                                       "context_lens", "scale", "split_k"]
    assert decode.parameters["scale"].kind is inspect.Parameter.KEYWORD_ONLY
    prefill = inspect.signature(tpa.triton_paged_prefill)
    assert list(prefill.parameters) == ["query", "key_cache", "value_cache", "cu_seqlens_q",
                                        "cu_seqlens_k", "block_tables", "max_seqlen_q", "scale"]
    assert prefill.parameters["max_seqlen_q"].default is inspect.Parameter.empty


def test_select_split_k_is_the_references():
    # triton_paged_attention.py:342-349: 4 below 64 (request, head) programs.
    assert (tpa.DEFAULT_SPLIT_K, tpa.MIN_PROGRAMS) == (4, 64)
    assert tpa._select_split_k(1, 32) == 4
    assert tpa._select_split_k(3, 21) == 4
    assert tpa._select_split_k(2, 32) == 1
    assert tpa._select_split_k(32, 16) == 1


def _decode_inputs(dtype=torch.bfloat16, block=16, d=32):
    q = torch.zeros(2, 4, d, dtype=dtype)
    kc = torch.zeros(8, block, 2, d, dtype=dtype)
    return q, kc, kc.clone(), torch.zeros(2, 4, dtype=torch.int32), torch.ones(2, dtype=torch.int32)


@pytest.mark.parametrize("case, message", [
    ("ndim", "shape"), ("dtype-mismatch", "share"), ("host", "GPU"),
])
def test_decode_rejects_like_the_reference(case, message):
    q, kc, vc, tables, lens = _decode_inputs()
    if case == "ndim":
        q = q[0]
    elif case == "dtype-mismatch":
        q = q.float()
    with pytest.raises(ValueError, match=message):
        tpa.triton_paged_decode(q, kc, vc, tables, lens)


def test_empty_decode_returns_empty_like():
    q, kc, vc, tables, lens = _decode_inputs()
    out = tpa.triton_paged_decode(q[:0], kc, vc, tables[:0], lens[:0])
    assert out.shape == (0, 4, 32) and out.dtype == q.dtype


@pytest.mark.parametrize("case, message", [
    ("fp32", "FP16/BF16"), ("head-dim", "multiple of 16"), ("gqa", "divisible"),
    ("block", "power-of-two"), ("cu-q", "cu_seqlens_q"), ("cu-k", "cu_seqlens_k"),
    ("max-q", "positive"),
])
def test_prefill_rejects_like_the_reference(case, message):
    dtype, d, hq, block = torch.bfloat16, 32, 4, 16
    if case == "fp32":
        dtype = torch.float32
    if case == "head-dim":
        d = 24
    if case == "gqa":
        hq = 3
    if case == "block":
        block = 12
    q = torch.zeros(5, hq, d, dtype=dtype)
    kc = torch.zeros(8, block, 2, d, dtype=dtype)
    tables = torch.zeros(2, 4, dtype=torch.int32)
    cu_q = torch.tensor([0, 3, 5] if case != "cu-q" else [0, 5], dtype=torch.int32)
    cu_k = torch.tensor([0, 9, 20] if case != "cu-k" else [0, 20], dtype=torch.int32)
    with pytest.raises(ValueError, match=message):
        tpa.triton_paged_prefill(q, kc, kc.clone(), cu_q, cu_k, tables,
                                 max_seqlen_q=0 if case == "max-q" else 3)


def test_drop_ins_route_to_the_hip_ops():
    # Nothing but the HIP ops runs behind the reference names.
    source = inspect.getsource(tpa)
    assert "hip_paged_decode(" in source and "hip_paged_prefill(" in source
    assert tpa.hip_paged_decode is hip_paged_decode and tpa.hip_paged_prefill is hip_paged_prefill

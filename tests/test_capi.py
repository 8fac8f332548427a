"""The C-ABI library loads and exports what include/*.h declares.

No kernel is launched here: argument validation returns before any HIP call,
so these run on a host without a GPU.
"""

import ctypes
import re
from pathlib import Path

import pytest

from microinfer_amd import _lib

HEADERS = sorted((Path(__file__).resolve().parents[1] / "include").glob("*.h"))


def declared_functions():
    names = set()
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names |= set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(mi_\w+)\s*\(", text, re.M))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 8
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"


def test_abi_version_and_clean_error_state():
    lib = _lib.load()
    assert lib.mi_abi_version() == 102
    assert isinstance(_lib.last_error(), str)


def test_invalid_arguments_fail_before_launch():
    lib = _lib.load()
    status = lib.mi_kv_append(None, 0, 0, None, 0, 0, None, None, 0, 0, 0, None, None, 0,
                              1, 1, 8, 16, 4, 9, None)
    assert status == 1 and "dtype" in _lib.last_error()
    status = lib.mi_paged_decode(None, 0, 0, None, None, 0, 0, 0, None, 0, 1, None, None, 0, 0,
                                 None, 0, None, None, 0, 1, 3, 2, 128, 16, 4, 0, 1.0, 2, None)
    assert status == 1 and "multiple" in _lib.last_error()
    status = lib.mi_paged_decode(None, 0, 0, None, None, 0, 0, 0, None, 0, 1, None, None, 0, 0,
                                 None, 0, None, None, 0, 1, 4, 2, 96, 16, 4, 0, 1.0, 2, None)
    assert status == 2 and "head_dim" in _lib.last_error()
    status = lib.mi_paged_prefill(None, 0, 0, None, None, 0, 0, 0, None, None, None, 0, 1,
                                  None, 0, 0, 4, 1, 4, 4, 2, 128, 12, 4, 1.0, 2, None)
    assert status == 1 and "block_size" in _lib.last_error()
    status = lib.mi_gather_kv(None, None, 0, 0, 0, None, 0, 1, None, 0, 5, None, None, 2, 128,
                              16, 4, 2, None)
    assert status == 1 and "requests" in _lib.last_error()


def test_empty_work_is_a_no_op():
    lib = _lib.load()
    assert lib.mi_kv_append(None, 0, 0, None, 0, 0, None, None, 0, 0, 0, None, None, 0,
                            0, 8, 128, 16, 4, 2, None) == 0
    assert lib.mi_paged_decode(None, 0, 0, None, None, 0, 0, 0, None, 0, 1, None, None, 0, 0,
                               None, 0, None, None, 0, 0, 16, 8, 128, 16, 4, 0, 1.0, 2,
                               None) == 0


def test_missing_workspace_is_reported():
    lib = _lib.load()
    need = lib.mi_paged_decode_workspace_bytes(32, 16, 8, 128, 0)
    assert need > 0
    fake = ctypes.c_void_p(256)
    status = lib.mi_paged_decode(fake, 2048, 128, fake, fake, 16384, 1024, 128, fake, 128, 128,
                                 fake, fake, 2048, 128, None, 0, None, None, 0, 32, 16, 8, 128,
                                 16, 4096, 0, 1.0, 2, None)
    assert status == 3 and "workspace" in _lib.last_error()
    status = lib.mi_paged_decode(fake, 2048, 128, fake, fake, 16384, 1024, 128, fake, 128, 128,
                                 fake, fake, 2048, 128, fake, need, None, None, 0, 32, 16, 8, 128,
                                 16, 4096, 0, 1.0, 2, None)
    assert status == 3 and "counters" in _lib.last_error()
    # A plan buffer smaller than the current tuning needs is refused.
    status = lib.mi_paged_decode(fake, 2048, 128, fake, fake, 16384, 1024, 128, fake, 128, 128,
                                 fake, fake, 2048, 128, fake, need, fake, fake, 64, 32, 16, 8,
                                 128, 16, 4096, 0, 1.0, 2, None)
    assert status == 1 and "plan" in _lib.last_error()


def test_decode_plan_validation_and_size():
    lib = _lib.load()
    assert lib.mi_decode_plan_bytes(32, 8, 0) == (192 // 8 + 32) * 32
    assert lib.mi_decode_plan_bytes(4, 8, 16) == 4 * 16 * 32
    fake = ctypes.c_void_p(256)
    assert lib.mi_decode_plan(fake, 32, 8, 12, 128, 0, fake, 10 ** 6, None) == 1
    assert "block_size" in _lib.last_error()
    assert lib.mi_decode_plan(fake, 5000, 8, 16, 128, 0, fake, 10 ** 6, None) == 2
    assert lib.mi_decode_plan(fake, 32, 8, 16, 128, 0, fake, 64, None) == 3
    assert lib.mi_decode_plan(None, 0, 8, 16, 128, 0, None, 0, None) == 0


@pytest.mark.parametrize("split_k", [1, 0, 4])
def test_workspace_size_formula(split_k):
    lib = _lib.load()
    size = lib.mi_paged_decode_workspace_bytes(4, 32, 8, 128, split_k)
    plan = lib.mi_decode_plan_bytes(4, 8, split_k)
    plan_region = (plan + 255) // 256 * 256
    items = plan // 32
    partials = 0 if split_k == 1 else items * 8 * 4 * (128 + 2) * 4
    assert size == plan_region + partials


def test_prefill_workspace_size_and_refusal():
    lib = _lib.load()
    r256 = lambda x: (x + 255) // 256 * 256  # noqa: E731
    # bf16, 4120 rows in 32 requests, 32 Q / 8 KV heads: 1024 partial slots
    # (128 partitions x 8 KV heads) of 4 wave regions, 64 counters per KV head.
    regions = 128 * 8 * 4
    entries = (4120 + 31) // 32 + 32 + 128
    need = lib.mi_paged_prefill_workspace_bytes(4120, 32, 32, 8, 128, 2)
    assert need == (256 + r256(64 * 8 * 4) + r256(entries * 32) + r256(regions * 2 * 64 * 4)
                    + regions * 4096 * 4)
    assert lib.mi_paged_prefill_workspace_bytes(4120, 32, 32, 8, 128, 1) == need  # f16
    # No workspace where the call is not planned.
    assert lib.mi_paged_prefill_workspace_bytes(4120, 32, 32, 8, 128, 0) == 0  # f32
    assert lib.mi_paged_prefill_workspace_bytes(4120, 32, 32, 8, 64, 2) == 0
    assert lib.mi_paged_prefill_workspace_bytes(4120, 32, 64, 8, 128, 2) == 0  # group 8
    assert lib.mi_paged_prefill_workspace_bytes(8192, 4097, 32, 8, 128, 2) == 0
    fake = ctypes.c_void_p(256)
    args = [fake, 4096, 128, fake, fake, 16384, 1024, 128, fake, fake, fake, 256, 256,
            fake, 4096, 128, 4120, 32, 512, 32, 8, 128, 16, 65536, 0.088, 2]
    assert lib.mi_paged_prefill_planned(*args, fake, need - 1, 0, None) == 3
    assert "workspace" in _lib.last_error()
    misaligned = ctypes.c_void_p(256 + 16)
    assert lib.mi_paged_prefill_planned(*args, misaligned, need, 0, None) == 3
    assert lib.mi_paged_prefill_planned(*args, fake, need, 2, None) == 1  # unknown flag
    # The plan alone: the same sizes and workspace rules.
    plan_args = [fake, fake, 4120, 32, 32, 8, 128, 1, 16, 256, 65536, 2]
    assert lib.mi_paged_prefill_plan(*plan_args, fake, need - 1, None) == 3
    assert lib.mi_paged_prefill_plan(*plan_args[:-1], 0, fake, need, None) == 2  # f32
    bad_block = plan_args[:8] + [12] + plan_args[9:]
    assert lib.mi_paged_prefill_plan(*bad_block, fake, need, None) == 1


def test_dense_ops_validate_before_launch():
    lib = _lib.load()
    fake = ctypes.c_void_p(256)
    # n not a multiple of 16, k not a multiple of 32
    assert lib.mi_linear(fake, 1024, fake, 1024, fake, 1000, 8, 1000, 1024, 2, None) == 1
    assert lib.mi_linear(fake, 1000, fake, 1000, fake, 1024, 8, 1024, 1000, 2, None) == 1
    # more than 64 rows, or 32-bit elements: no kernel (the caller keeps torch)
    assert lib.mi_linear(fake, 1024, fake, 1024, fake, 1024, 65, 1024, 1024, 2, None) == 2
    assert lib.mi_linear(fake, 1024, fake, 1024, fake, 1024, 8, 1024, 1024, 0, None) == 2
    # strides below the row lengths, misaligned rows
    assert lib.mi_linear(fake, 512, fake, 1024, fake, 1024, 8, 1024, 1024, 2, None) == 1
    assert lib.mi_linear(fake, 1028, fake, 1024, fake, 1024, 8, 1024, 1024, 2, None) == 1
    assert "aligned" in _lib.last_error()
    assert lib.mi_linear(None, 0, None, 0, None, 0, 0, 1024, 1024, 2, None) == 0
    assert lib.mi_rms_norm_residual(fake, 1024, None, 0, fake, 1e-6, fake, 1024, None, 0, 4,
                                    1020, 2, None) == 1
    assert lib.mi_rms_norm_residual(fake, 1024, None, 0, fake, 1e-6, fake, 1024, None, 0, 4,
                                    1024, 0, None) == 2
    assert lib.mi_rms_norm_residual(fake, 16384, None, 0, fake, 1e-6, fake, 16384, None, 0, 4,
                                    16384, 2, None) == 2
    assert lib.mi_rms_norm_residual(None, 0, None, 0, None, 1e-6, None, 0, None, 0, 0, 1024,
                                    2, None) == 0
    assert lib.mi_silu_mul(fake, 6144, fake, 3072, 4, 3070, 2, None) == 1
    assert lib.mi_silu_mul(fake, 6000, fake, 3072, 4, 3072, 2, None) == 1
    assert lib.mi_silu_mul(None, 0, None, 0, 0, 3072, 2, None) == 0
    # fused gate/up + SwiGLU: inter not a multiple of 16, output stride below
    # inter, more than 64 rows, an empty batch
    assert lib.mi_linear_swiglu(fake, 1024, fake, 1024, fake, 3072, 8, 3064, 1024, 2, None) == 1
    assert lib.mi_linear_swiglu(fake, 1024, fake, 1024, fake, 3000, 8, 3072, 1024, 2, None) == 1
    assert lib.mi_linear_swiglu(fake, 1024, fake, 1024, fake, 3072, 65, 3072, 1024, 2, None) == 2
    assert lib.mi_linear_swiglu(None, 0, None, 0, None, 0, 0, 3072, 1024, 2, None) == 0


def test_noalloc_refuses_calls_beyond_its_scratch():
    # The size check returns before any HIP call (no device lookup, no
    # launch), so the placeholder pointers are never dereferenced.
    lib = _lib.load()
    room = lib.mi_paged_decode_noalloc_max_bytes()
    assert room > 0
    # 4096 sequences of a 128-query-head layer need far more than the scratch.
    assert lib.mi_paged_decode_workspace_bytes(4096, 128, 16, 256, 0) > room
    fake = 256
    status = lib.mi_paged_decode_append_noalloc(
        fake, 4096, 256, fake, 4096, 256, fake, 32768, 256, fake, fake, 65536, 4096, 256,
        fake, 1, 1, fake, fake, 32768, 256, 4096, 128, 16, 256, 16, 64, 0, 1.0, 2, None)
    assert status == 3 and "scratch" in _lib.last_error()

"""Bit-level helpers for 16-bit floats on the CPU (test infrastructure only).

numpy has no bfloat16, so bf16 tensors travel as ``uint16`` bit patterns.
bf16 -> fp32 is exact (append 16 zero bits). fp32 -> bf16 is round to nearest
even with a canonical quiet NaN (0x7FC0), which is the rounding PyTorch's
``c10::BFloat16`` uses for ``tensor.to(torch.bfloat16)``; fp16 uses numpy's
IEEE round-to-nearest-even cast, as PyTorch does.

Pinned by: tests/test_oracle_numerics.py (exhaustive round trip of all 65536
bf16 patterns, hand-checked tie cases, agreement with torch's own CPU cast on
random and edge inputs).
"""

from __future__ import annotations

import numpy as np


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact widening of bf16 bit patterns (uint16) to float32."""
    bits = np.asarray(bits, dtype=np.uint16)
    return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16_bits(values: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even, NaN -> 0x7FC0."""
    values = np.ascontiguousarray(values, dtype=np.float32)
    u = values.view(np.uint32).astype(np.uint64)
    rounding_bias = ((u >> np.uint64(16)) & np.uint64(1)) + np.uint64(0x7FFF)
    rounded = ((u + rounding_bias) >> np.uint64(16)).astype(np.uint16)
    return np.where(np.isnan(values), np.uint16(0x7FC0), rounded).astype(np.uint16)


def round_to_dtype(values: np.ndarray, dtype: str) -> np.ndarray:
    """Round float values to ``dtype`` and return them widened to float32.

    ``dtype`` is one of "f32", "f16", "bf16". The result is what a kernel that
    stores ``dtype`` and reads it back as float32 would see.
    """
    values = np.asarray(values, dtype=np.float32)
    if dtype == "f32":
        return values.copy()
    if dtype == "f16":
        return values.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        return bf16_bits_to_f32(f32_to_bf16_bits(values))
    raise ValueError(f"unknown dtype {dtype!r}")

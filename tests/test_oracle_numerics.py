"""Pin the oracle's bf16/fp16 bit helpers."""

import numpy as np
import torch

from oracle.numerics import bf16_bits_to_f32, f32_to_bf16_bits, round_to_dtype


def test_every_bf16_pattern_round_trips():
    patterns = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    widened = bf16_bits_to_f32(patterns)
    back = f32_to_bf16_bits(widened)
    nan = np.isnan(widened)
    assert np.array_equal(back[~nan], patterns[~nan])
    assert (back[nan] == 0x7FC0).all()


def test_ties_round_to_even():
    # 1 + 2^-8 sits halfway between bf16 1.0 (0x3F80) and 1 + 2^-7 (0x3F81).
    half_up = np.array([1 + 2.0**-8, 1 + 3 * 2.0**-8, -(1 + 2.0**-8)], dtype=np.float32)
    assert f32_to_bf16_bits(half_up).tolist() == [0x3F80, 0x3F82, 0xBF80]
    # Just above the tie rounds up.
    above = np.array([np.nextafter(np.float32(1 + 2.0**-8), np.float32(2))], dtype=np.float32)
    assert f32_to_bf16_bits(above).tolist() == [0x3F81]


def test_matches_torch_cast():
    rng = np.random.default_rng(0)
    values = np.concatenate(
        [
            rng.standard_normal(4096).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 4096),
            np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, -3.4e38, 1e-40, -1e-45], np.float32),
        ]
    ).astype(np.float32)
    expected = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy()
    assert np.array_equal(f32_to_bf16_bits(values).view(np.int16), expected)
    half = torch.from_numpy(values).to(torch.float16).float().numpy()
    np.testing.assert_array_equal(round_to_dtype(values, "f16"), half)
    bf = torch.from_numpy(values).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(round_to_dtype(values, "bf16"), bf)

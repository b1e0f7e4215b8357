"""Pins the oracle's bf16 rounding against torch's own fp32 -> bf16 conversion."""

import numpy as np
import torch

from oracle.bf16 import R, to_bf16, to_f32, ulp_distance


def _torch_bits(values: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(values.astype(np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def test_matches_torch_on_random_values():
    rng = np.random.default_rng(0)
    values = np.concatenate([
        rng.standard_normal(100_000) * 10.0 ** rng.integers(-30, 30, 100_000),
        rng.standard_normal(10_000),
    ]).astype(np.float32)
    assert np.array_equal(to_bf16(values), _torch_bits(values))


def test_ties_round_to_even_and_specials():
    # Exact halfway points between consecutive bf16 values, both parities.
    halfway = np.array([0x3F808000, 0x3F818000, 0xBF808000, 0xBF818000], dtype=np.uint32)
    values = np.concatenate([
        halfway.view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.4e38, -3.4e38], np.float32),
    ])
    assert np.array_equal(to_bf16(values), _torch_bits(values))
    assert to_bf16(np.array([np.nan], np.float32))[0] == 0x7FC0


def test_round_trip_is_identity_on_bf16_values():
    bits = np.arange(0, 0x10000, dtype=np.uint32).astype(np.uint16)
    finite = (bits & 0x7F80) != 0x7F80
    assert np.array_equal(to_bf16(to_f32(bits[finite])), bits[finite])


def test_R_is_one_rounding_and_ulp_distance_counts_steps():
    a = to_bf16(np.array([1.0], np.float32))
    b = np.array([a[0] + 3], np.uint16)
    assert ulp_distance(a, b)[0] == 3
    # +0 and -0 are the same value: zero steps apart.
    assert ulp_distance(np.array([0x0000], np.uint16), np.array([0x8000], np.uint16))[0] == 0
    assert R(np.array([1.0 + 2**-9], np.float32))[0] == 1.0

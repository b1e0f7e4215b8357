"""Helpers shared by the tests: seeded bf16 inputs and host/device bit transfers."""

from __future__ import annotations

import numpy as np
import torch

from oracle.bf16 import from_float, to_f32, ulp_distance

BF16_ULP = 2.0**-8


def bf16_normal(rng: np.random.Generator, shape, scale: float = 1.0, shift: float = 0.0):
    return from_float(shift + scale * rng.standard_normal(shape))


def to_device(bits: np.ndarray, device: str = "cuda") -> torch.Tensor:
    """uint16 bf16 bits -> torch bf16 tensor on `device`."""
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)
    return t.to(device)


def f32_to_device(values: np.ndarray, device: str = "cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(values, dtype=np.float32)).to(device)


def bits_of(t: torch.Tensor) -> np.ndarray:
    """torch bf16 tensor -> uint16 bit pattern array on the host."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def relative_diff(got, want) -> float:
    """The reference's house metric (tests/conftest.py:49-59): max|a - b| / max|b| in fp32."""
    a = np.asarray(got, dtype=np.float64)
    b = np.asarray(want, dtype=np.float64)
    scale = np.abs(b).max() if b.size else 0.0
    return float(np.abs(a - b).max() / scale) if b.size and scale > 0 else 0.0


def assert_bf16_close(got_bits, want_bits, *, max_ulp: int = 2, atol=1e-2, rtol=1e-2,
                      min_exact: float = 0.999):
    """The bf16 output bar against the oracle.

    - every element within atol/rtol 1e-2 after widening;
    - the house metric max|a-b|/max|b| within `max_ulp` bf16 ulps (2 * 2^-8): an ulp
      distance per element is not used as a bound because an output that cancels to
      near zero (a*cos - b*sin) has a tiny ulp, so a one-ulp difference in one input
      reads as many ulps there while staying small in absolute terms;
    - at least `min_exact` of the elements bit-identical, so a systematic slip (a wrong
      index or rounding point) cannot hide inside the tolerance.
    Returns the per-element ulp distances.
    """
    got_bits = np.asarray(got_bits)
    want_bits = np.asarray(want_bits)
    assert got_bits.shape == want_bits.shape, (got_bits.shape, want_bits.shape)
    got, want = to_f32(got_bits), to_f32(want_bits)
    np.testing.assert_allclose(got, want, atol=atol, rtol=rtol)
    diff = relative_diff(got, want)
    assert diff <= max_ulp * BF16_ULP, f"relative_diff {diff:.3g} > {max_ulp} bf16 ulp"
    dist = ulp_distance(got_bits, want_bits)
    exact = float(np.mean(dist == 0)) if dist.size else 1.0
    assert exact >= min_exact, f"only {exact:.5f} bit-identical ({int((dist > 0).sum())} differ)"
    return dist


def exact_fraction(got_bits, want_bits) -> float:
    got_bits = np.asarray(got_bits)
    return float(np.mean(got_bits == np.asarray(want_bits))) if got_bits.size else 1.0

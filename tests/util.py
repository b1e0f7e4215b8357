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


def assert_bf16_close(got_bits, want_bits, *, max_ulp: int = 2, atol=1e-2, rtol=1e-2):
    """The bf16 output bar: within `max_ulp` ulps and within atol/rtol after widening."""
    got_bits = np.asarray(got_bits)
    want_bits = np.asarray(want_bits)
    assert got_bits.shape == want_bits.shape, (got_bits.shape, want_bits.shape)
    dist = ulp_distance(got_bits, want_bits)
    worst = int(dist.max()) if dist.size else 0
    assert worst <= max_ulp, f"{worst} ulp apart (max {max_ulp}); {int((dist > 0).sum())} differ"
    np.testing.assert_allclose(to_f32(got_bits), to_f32(want_bits), atol=atol, rtol=rtol)
    return dist


def exact_fraction(got_bits, want_bits) -> float:
    got_bits = np.asarray(got_bits)
    return float(np.mean(got_bits == np.asarray(want_bits))) if got_bits.size else 1.0

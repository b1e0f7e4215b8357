"""bf16 <-> fp32 as bit operations (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

`to_bf16` is IEEE round-to-nearest-even on the fp32 bit pattern — the rounding MLX's
`astype(bfloat16)` and every bf16 op output perform (the `T(...)` casts in the reference
kernels, e.g. core/kernels/add_norm/rows.py:65-79). NaN maps to the canonical quiet NaN
0x7FC0.
"""

from __future__ import annotations

import numpy as np


def to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32 values (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_bf16(values: np.ndarray) -> np.ndarray:
    """float32 values -> bf16 bit patterns with round-to-nearest-even."""
    f = np.ascontiguousarray(values, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (f.view(np.uint32) & 0x7FFFFFFF) > 0x7F800000
    rounded[nan] = 0x7FC0
    return rounded


def R(values: np.ndarray) -> np.ndarray:
    """One bf16 rounding step, result widened back to float32."""
    return to_f32(to_bf16(values))


def from_float(values) -> np.ndarray:
    """Any real array -> float32 -> bf16 bits (how seeded inputs are made)."""
    return to_bf16(np.asarray(values, dtype=np.float32))


def ulp_distance(a_bits: np.ndarray, b_bits: np.ndarray) -> np.ndarray:
    """Distance in bf16 ulps between two bf16 bit arrays (monotone integer map)."""
    def ordinal(bits):
        b = np.asarray(bits, dtype=np.uint16).astype(np.int32)
        return np.where(b & 0x8000, 0x8000 - (b & 0x7FFF), 0x8000 + b)
    return np.abs(ordinal(a_bits) - ordinal(b_bits))

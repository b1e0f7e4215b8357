"""Residual add + RMSNorm (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

Restates core/kernels/add_norm/default.py:28-29 (`added = x + p`, then
`mx.fast.rms_norm(added, w, eps)`) with the rounding points mx.fast.rms_norm uses and
core/kernels/add_norm/rows.py:65-79 copies:

    s_i = R(x_i + p_i)
    inv = 1 / sqrt(sum_i s_i^2 / H + eps)
    n_i = R(w_i * R(s_i * inv))

The sum of squares is taken in float64 and rounded to float32 once: the correctly
rounded fp32 sum, one admissible result of the fp32 accumulation whose order the
reference leaves free (and the one the HIP kernels produce, since they accumulate the
exact bf16 squares in fp64). Every later step is float32, operation for operation.
"""

from __future__ import annotations

import numpy as np

from .bf16 import R, to_bf16, to_f32


def inverse_rms(s: np.ndarray, eps: float) -> np.ndarray:
    """`1 / sqrt(mean(s^2) + eps)` over the last axis of float32 values -> float32 [..., 1]."""
    hidden = np.float32(s.shape[-1])
    total = np.sum(s.astype(np.float64) ** 2, axis=-1, keepdims=True).astype(np.float32)
    mean = total / hidden
    return np.float32(1.0) / np.sqrt(mean + np.float32(eps))


def rms_norm(x_bits: np.ndarray, w_bits: np.ndarray, eps: float) -> np.ndarray:
    """mx.fast.rms_norm on bf16 rows (core/kernels/add_norm/rows.py:75-79)."""
    s = to_f32(x_bits)
    inv = inverse_rms(s, eps)
    return to_bf16(to_f32(w_bits) * R(s * inv))


def add_rms_norm(
    x_bits: np.ndarray, branch_bits: np.ndarray, w_bits: np.ndarray, eps: float
) -> tuple[np.ndarray, np.ndarray]:
    """(summed, normalized) bf16 bits; core/kernels/add_norm/default.py:28-29."""
    summed = to_bf16(to_f32(x_bits) + to_f32(branch_bits))
    return summed, rms_norm(summed, w_bits, eps)

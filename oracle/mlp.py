"""Dense SwiGLU MLP of one token, bf16 weights (TEST INFRASTRUCTURE ONLY; see
oracle/__init__.py).

Restates the reference's two-dispatch `DenseMlp` (core/kernels/mlp/dense.py:34-147,
222-246):

- gate_up_swiglu (:34-97): g = T(sum_h x_h * W[n, h]), u = T(sum_h x_h * W[I + n, h]),
  the projections evaluated in float64 and rounded once to bf16 (the exact dot product
  for all practical purposes, which the reference's fp32 sweep approximates); then the
  stable exp(|g|) chain with every temporary a bf16 value (:86-96):
      e = T(exp(|g|)), den = T(1 + e), y = T(1 / den), sig = g < 0 ? y : T(1 - y),
      act = T(T(g * sig) * u)
  exp is evaluated in float64 and rounded once; every other step is the float32
  operation on bf16 operands, rounded (a bf16 value computed in float, as `bfloat`
  arithmetic is).
- down_residual (:100-147): out[n] = T(residual[n] + T(sum_i act_i * D[n, i])), the dot
  product in float64 rounded once, the add in float32.
"""

from __future__ import annotations

import numpy as np

from .activations import f64_to_bf16
from .bf16 import R, to_bf16, to_f32


def swiglu_steps(gate_bits: np.ndarray, up_bits: np.ndarray) -> np.ndarray:
    """The bf16 SwiGLU chain of core/kernels/mlp/dense.py:86-96 on bf16 inputs."""
    g = to_f32(gate_bits)
    u = to_f32(up_bits)
    with np.errstate(over="ignore"):
        e = to_f32(f64_to_bf16(np.exp(np.abs(g).astype(np.float64))))
    one = np.float32(1.0)
    den = R(one + e)
    with np.errstate(divide="ignore"):
        y = R(one / den)
    sig = np.where(g < 0, y, R(one - y)).astype(np.float32)
    silu = R(g * sig)
    return to_bf16(silu * u)


def project(x_bits: np.ndarray, weight_bits: np.ndarray) -> np.ndarray:
    """bf16 rows [n, k] times a bf16 vector [k] -> [n] bf16 bits, one rounding."""
    x = to_f32(np.asarray(x_bits).reshape(-1)).astype(np.float64)
    return f64_to_bf16(to_f32(weight_bits).astype(np.float64) @ x)


def gate_up_swiglu(x_bits: np.ndarray, fused_bits: np.ndarray) -> np.ndarray:
    """x [hidden] bf16 bits, fused weight [2 * inner, hidden] bf16 bits (gate rows first)
    -> [inner] bf16 bits."""
    projected = project(x_bits, fused_bits)
    inner = fused_bits.shape[0] // 2
    return swiglu_steps(projected[:inner], projected[inner:])


def down_residual(act_bits: np.ndarray, down_bits: np.ndarray, residual_bits: np.ndarray) -> np.ndarray:
    """act [inner] bf16 bits, down weight [hidden, inner] bf16 bits, residual [hidden] bf16
    bits -> [hidden] bf16 bits."""
    down = to_f32(project(act_bits, down_bits))
    return to_bf16(to_f32(np.asarray(residual_bits).reshape(-1)) + down)


def mlp(x_bits, fused_bits, down_bits, residual_bits) -> np.ndarray:
    """Both dispatches: the activation handed from the first to the second in bf16."""
    return down_residual(gate_up_swiglu(x_bits, fused_bits), down_bits, residual_bits)

"""SwiGLU and gate-softplus (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

SwiGLU restates the Core chain `gate * mx.sigmoid(gate) * up` (core/layers.py:249-250,
284-287; core/kernels/gate_up/default.py:71-81) as three bf16 ops, each rounding its
result:  s = R(sigmoid(g)),  t = R(g * s),  y = R(t * u).  The sigmoid is evaluated in
float64 and rounded once, straight to bf16 (the correctly rounded value); g * s and
t * u are exact in float32 (products of two bf16 values) before their rounding.

Gate-softplus restates models/qwen3_5/layers/deltanet.py:222-224:
    dt = f32(a) + dt_bias;  g = -exp(A_log) * softplus(dt)
with nn.softplus = mx.logaddexp(dt, 0) = max + log1p(exp(min - max)) and its arms
(min == -inf or max == inf -> max), every float32 step correctly rounded (evaluated in
float64, rounded once to float32).
"""

from __future__ import annotations

import numpy as np

from .bf16 import to_bf16, to_f32


def f64_to_bf16(values: np.ndarray) -> np.ndarray:
    """float64 -> bf16 bits with one round-to-nearest-even (no float32 step) for values
    in the normal bf16 range; others (zero, subnormal, inf, NaN) go through float32."""
    v = np.ascontiguousarray(values, dtype=np.float64)
    bits = v.view(np.uint64)
    sign = ((bits >> np.uint64(48)) & np.uint64(0x8000)).astype(np.uint32)
    exponent = ((bits >> np.uint64(52)) & np.uint64(0x7FF)).astype(np.int64) - 1023
    mantissa = bits & np.uint64((1 << 52) - 1)
    rest = mantissa & np.uint64((1 << 45) - 1)
    half = np.uint64(1 << 44)
    magnitude = (((exponent + 127).clip(0, 255).astype(np.uint32)) << 7) | (
        mantissa >> np.uint64(45)).astype(np.uint32)
    bump = (rest > half) | ((rest == half) & ((magnitude & 1) == 1))
    out = (sign | (magnitude + bump.astype(np.uint32))).astype(np.uint16)
    normal = (exponent >= -126) & (exponent <= 127)
    return np.where(normal, out, to_bf16(v.astype(np.float32)))


def sigmoid_bf16(g: np.ndarray) -> np.ndarray:
    """Correctly rounded bf16 of sigmoid(g) (bits), g float32 values."""
    g64 = g.astype(np.float64)
    e = np.exp(-np.abs(g64))
    s = np.where(g64 >= 0, 1.0, e) / (1.0 + e)
    return f64_to_bf16(s)


def swiglu(gate_bits: np.ndarray, up_bits: np.ndarray) -> np.ndarray:
    g = to_f32(gate_bits)
    u = to_f32(up_bits)
    s = to_f32(sigmoid_bf16(g))
    with np.errstate(invalid="ignore"):  # -inf * sigmoid(-inf) = -inf * 0 is NaN, as on the device
        t = to_f32(to_bf16(g * s))
        return to_bf16(t * u)


def softplus_f32(dt: np.ndarray) -> np.ndarray:
    """mx.logaddexp(dt, 0) with correctly rounded float32 steps."""
    dt = np.asarray(dt, dtype=np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        maxval = np.where(dt > 0, dt, np.float32(0))
        minval = np.where(dt > 0, np.float32(0), dt)
        r1 = np.exp((minval - maxval).astype(np.float64)).astype(np.float32)
        r2 = np.log1p(r1.astype(np.float64)).astype(np.float32)
        sp = maxval + r2
    arms = (minval == -np.inf) | (maxval == np.inf)
    return np.where(arms, maxval, sp).astype(np.float32)


def gate_softplus(a_bits: np.ndarray, a_log: np.ndarray, dt_bias: np.ndarray) -> np.ndarray:
    dt = to_f32(a_bits) + dt_bias.astype(np.float32)
    decay = -(np.exp(a_log.astype(np.float64)).astype(np.float32))
    return (decay * softplus_f32(dt)).astype(np.float32)

"""Routed expert MLP of one token over MXFP4 expert stacks (TEST INFRASTRUCTURE ONLY;
see oracle/__init__.py).

Format: MLX's mode "mxfp4", the `QuantizedSwitchLinear` leaf (core/layers.py:164-197),
as core/kernels/shared/mxfp4.py:8-32 decodes it:

- weight [E, out, in / 8] uint32: two e2m1 codes per byte, the low nibble first, so
  value j of a row is nibble j of its little-endian bytes;
- e2m1 code (sign, e, m): (-1)^sign * (m / 2) when e = 0, else (-1)^sign * 2^(e - 1) *
  (1 + m / 2): 0, 0.5, 1, 1.5, 2, 3, 4, 6 and their negatives;
- scales [E, out, in / 32] uint8, e8m0: the group's factor is the fp32 whose bit pattern
  is `byte << 23` (2^(byte - 127) for bytes 1..254, 0 for byte 0);
- the projection's bias [E, out] bf16.

gate_up (core/kernels/gate_up/mxfp4.py:24-65), interleaved rows, swiglu_oai with its
clamp; every step rounds to T as written there:

    r   = sum over groups of scale * sum_j x_j v_j          fp32 there; float64 here
    g   = T(r_gate + b_gate), u = T(r_up + b_up)
    g   = T(min(g, limit)), u = T(clamp(u, -limit, limit))
    sig = T(1 / (1 + exp(-1.702 g)))                          each op in fp32
    y   = T(T(g * sig) * T(u + 1))

down_combine (core/kernels/down_combine/mxfp4.py:16-58):

    t   = the same dot product over inner                     float64 here
    acc = sum over slots in order of T(fp32(T(t + b) * w))    fp32
    y   = T(fp32(T(acc) + residual))

An expert id outside [0, experts) contributes zero rows (the HIP kernels' guard).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .bf16 import from_float, to_f32

E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                 -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])


@dataclass
class Stack:
    weight: np.ndarray   # uint32 [..., out, in / 8]
    scales: np.ndarray   # uint8 [..., out, in / 32]
    bias: np.ndarray     # bf16 bits [..., out], or None


def codes(weight: np.ndarray) -> np.ndarray:
    """uint32 words [..., n] -> e2m1 codes [..., 8 n], nibble j of the little-endian bytes."""
    b = np.ascontiguousarray(weight, dtype="<u4").view(np.uint8)
    return np.stack([b & 0xF, b >> 4], axis=-1).reshape(*b.shape[:-1], -1)


def scale_values(scales: np.ndarray) -> np.ndarray:
    """e8m0 bytes -> float64 factors: the fp32 with exponent field `byte`."""
    return (np.asarray(scales, dtype=np.uint32) << 23).view(np.float32).astype(np.float64)


def dequantize(stack: Stack) -> np.ndarray:
    """float64 [..., out, in] weights."""
    v = E2M1[codes(stack.weight)]
    s = np.repeat(scale_values(stack.scales), 32, axis=-1)
    return v * s


def pack(code_values: np.ndarray) -> np.ndarray:
    """e2m1 codes [..., n] (n a multiple of 8) -> uint32 words."""
    c = np.asarray(code_values, dtype=np.uint8)
    b = (c[..., 0::2] | (c[..., 1::2] << 4)).astype(np.uint8)
    return np.ascontiguousarray(b).view("<u4").astype(np.uint32)


def _slot(stack: Stack, e: int) -> tuple[np.ndarray, np.ndarray]:
    """(matrix float64, bias float32) of expert e; zeros for an invalid id."""
    experts, out = stack.weight.shape[0], stack.weight.shape[1]
    if not 0 <= e < experts:
        return np.zeros((out, stack.weight.shape[2] * 8)), np.zeros(out, dtype=np.float32)
    m = dequantize(Stack(stack.weight[e], stack.scales[e], None))
    b = np.zeros(out, dtype=np.float32) if stack.bias is None else to_f32(stack.bias[e])
    return m, b


def _T(values) -> np.ndarray:
    return to_f32(from_float(np.asarray(values, dtype=np.float32)))


def gate_up(x_bits: np.ndarray, stack: Stack, chosen, limit: float | None) -> np.ndarray:
    """x [H] bf16 bits, stack [E, 2I, ...] -> [slots, I] bf16 bits."""
    x = to_f32(np.asarray(x_bits).reshape(-1)).astype(np.float64)
    out = []
    for e in np.asarray(chosen).reshape(-1):
        m, b = _slot(stack, int(e))
        r = m @ x   # the kernels' fp32 sum, exact here; with the bias it rounds once to T
        g = _T((r[0::2] + b[0::2]).astype(np.float32))
        u = _T((r[1::2] + b[1::2]).astype(np.float32))
        out.append(swiglu_oai(g, u, limit))
    return np.stack(out)


def swiglu_oai(g: np.ndarray, u: np.ndarray, limit: float | None) -> np.ndarray:
    """The clamped activation on bf16-valued g and u, each step rounded to T -> bf16 bits."""
    if limit is not None:
        g = _T(np.minimum(g, np.float32(limit)))
        u = _T(np.clip(u, np.float32(-limit), np.float32(limit)))
    with np.errstate(over="ignore"):
        e = np.exp((np.float32(-1.702) * g).astype(np.float32), dtype=np.float32)
    sig = _T((np.float32(1.0) / (np.float32(1.0) + e)).astype(np.float32))
    act = _T(g * sig)
    return from_float(act * _T(u + np.float32(1.0)))


def down_combine(act_bits: np.ndarray, stack: Stack, chosen, weights,
                 residual_bits: np.ndarray | None) -> np.ndarray:
    """act [slots, I] bf16 bits, stack [E, H, ...], weights [slots] fp32 -> [H] bf16 bits."""
    chosen = np.asarray(chosen).reshape(-1)
    act = to_f32(np.asarray(act_bits).reshape(len(chosen), -1)).astype(np.float64)
    weights = np.asarray(weights, dtype=np.float32).reshape(-1)
    acc = np.zeros(stack.weight.shape[1], dtype=np.float32)
    for j, e in enumerate(chosen):
        valid = 0 <= int(e) < stack.weight.shape[0]
        m, b = _slot(stack, int(e))
        t = (m @ act[j])
        tb = _T((t + b).astype(np.float32)).astype(np.float64)
        term = _T((tb * np.float64(weights[j])).astype(np.float32)) if valid else np.zeros_like(acc)
        acc = (acc + term).astype(np.float32)
    out = _T(acc)
    if residual_bits is not None:
        out = (out + to_f32(np.asarray(residual_bits).reshape(-1))).astype(np.float32)
    return from_float(out)

"""Routed expert MLP of one token, dense bf16 weights (TEST INFRASTRUCTURE ONLY; see
oracle/__init__.py).

Restates the arithmetic of the dense bindings of the two T=1 expert primitives, under the
"blocked" layout (gate and up block-concatenated, the activation owned by the down half):

- gate_up (core/kernels/gate_up/dense.py:30-58): y[j, n] = T(sum_h x_h * W[c_j, n, h]).
  The reference accumulates in fp32 in a lane-sweep order of its own; here the dot
  product is evaluated in float64 and rounded once to bf16 (its exact value for all
  practical purposes, which any fp32 order approximates).
- down (core/kernels/down_combine/dense.py:21-52,109): per element of the pair block,
  a = g / (1 + exp(-g)) * u in fp32, each operation rounded to fp32 as the Metal source
  writes it; t = sum_i a_i * W[c_j, n, i] (float64 here, rounded to fp32);
  d[j, n] = T(fp32(t * w_j)); then the `routed.sum(axis=0) + residual` ops in bf16:
  out = T(T(sum_j d[j, n]) + residual[n]), the expert sum in fp32 in order j = 0, 1, ...

An expert id outside [0, experts) contributes a zero row (the HIP kernels' guard; the
reference reads whatever the index addresses).
"""

from __future__ import annotations

import numpy as np

from .activations import f64_to_bf16
from .bf16 import from_float, to_f32


def _rows(weight_bits: np.ndarray, chosen: np.ndarray) -> np.ndarray:
    """Gathered expert matrices as float64 [k, out, in]; invalid ids give zeros."""
    chosen = np.asarray(chosen, dtype=np.int64)
    experts = weight_bits.shape[0]
    valid = (chosen >= 0) & (chosen < experts)
    rows = to_f32(weight_bits[np.where(valid, chosen, 0)]).astype(np.float64)
    rows[~valid] = 0.0
    return rows


def gate_up(x_bits: np.ndarray, weight_bits: np.ndarray, chosen: np.ndarray) -> np.ndarray:
    """x [H] bf16 bits, weight [E, 2I, H] bf16 bits, chosen [k] -> [k, 2I] bf16 bits."""
    x = to_f32(x_bits.reshape(-1)).astype(np.float64)
    return f64_to_bf16(_rows(weight_bits, chosen) @ x)


def swiglu_fp32(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """g / (1 + exp(-g)) * u with every operation rounded to fp32 (the Metal expression)."""
    g = gate.astype(np.float32)
    with np.errstate(over="ignore"):
        e = np.exp(-g, dtype=np.float32)
    den = (np.float32(1.0) + e).astype(np.float32)
    return ((g / den).astype(np.float32) * up.astype(np.float32)).astype(np.float32)


def down_combine(act_bits: np.ndarray, weight_bits: np.ndarray, chosen: np.ndarray,
                 weights: np.ndarray, residual_bits: np.ndarray | None) -> np.ndarray:
    """act [k, 2I] bf16 bits, weight [E, H, I] bf16 bits, chosen [k], weights [k] fp32,
    residual [H] bf16 bits or None -> [H] bf16 bits."""
    k = len(chosen)
    inner = weight_bits.shape[2]
    block = to_f32(act_bits.reshape(k, 2 * inner))
    a = swiglu_fp32(block[:, :inner], block[:, inner:]).astype(np.float64)
    t = np.einsum("kni,ki->kn", _rows(weight_bits, chosen), a).astype(np.float32)
    d = to_f32(from_float((t * np.asarray(weights, dtype=np.float32)[:, None]).astype(np.float32)))
    chosen = np.asarray(chosen, dtype=np.int64)
    d[(chosen < 0) | (chosen >= weight_bits.shape[0])] = 0.0
    total = np.zeros(weight_bits.shape[1], dtype=np.float32)
    for j in range(k):
        total = (total + d[j]).astype(np.float32)
    out = to_f32(from_float(total))
    if residual_bits is not None:
        out = (out + to_f32(residual_bits.reshape(-1))).astype(np.float32)
    return from_float(out)

"""Routed expert MLP of one token over affine-quantized expert stacks (TEST INFRASTRUCTURE
ONLY; see oracle/__init__.py).

Format: MLX's affine quantization, the `QuantizedSwitchLinear` leaf
(core/layers.py:164-197, `mode="affine"`), decoded as core/kernels/shared/affine.py:9-58
reads it:

- weight [E, out, in * bits / 32] uint32. A row is one little-endian bit stream: value j
  sits at bit offset j * bits (bits 0..3 of word 0 hold value 0 at 4 bits, and a value
  may straddle two words at 3, 5 and 6 bits);
- scales, biases [E, out, in / group] bf16;
- w[o, j] = scale[o, j // group] * q[o, j] + bias[o, j // group].

gate_up (core/kernels/gate_up/affine.py:24-95), the interleaved layout (row 2n is the gate
of output n, row 2n + 1 its up), silu:

    r   = sum_groups(scale * sum_j x_j q_j + bias * sum_j x_j)    fp32 there; float64 here
    g   = T(r_gate), u = T(r_up); with a limit, g = min(g, limit), u = clip(u, -limit, limit)
    sg  = T(1 / (1 + exp(-g)))                                     each op in fp32
    y   = T(T(g * sg) * u)

down_combine (core/kernels/down_combine/affine.py:17-70), over the activation rows:

    t_e = the same dot product over inner                          fp32 there; float64 here
    acc = sum over slots e, in order, of T(fp32(T(t_e) * w_e))     fp32
    y   = T(fp32(T(acc) + residual))

With a shared expert declared, the last slot reads the shared leaf (2-D, its own width and
group) and its index is not read (gate_up/affine.py:36-49, down_combine/affine.py:29-44).
An expert id outside [0, experts) gives a zero row (the HIP kernels' guard; the reference
reads whatever the index addresses).

The dot products are exact in float64 and rounded once, the value every fp32 order
approximates; `quantize` is a plain min/max affine quantizer that makes test stacks (the
kernels read whatever (q, scale, bias) they are given, so the quantizer's own rounding is
not part of the contract).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .activations import f64_to_bf16
from .bf16 import from_float, to_f32

WIDTHS = (2, 3, 4, 5, 6, 8)
GROUPS = (32, 64, 128)


@dataclass
class Stack:
    """One affine-quantized leaf: [E, out, in] (or [out, in] for a shared expert)."""

    weight: np.ndarray   # uint32 [..., out, in * bits / 32]
    scales: np.ndarray   # bf16 bits [..., out, in / group]
    biases: np.ndarray   # bf16 bits [..., out, in / group]
    group: int
    bits: int

    @property
    def in_features(self) -> int:
        return self.weight.shape[-1] * 32 // self.bits


def unpack(weight: np.ndarray, bits: int) -> np.ndarray:
    """uint32 words [..., words] -> integer values [..., words * 32 / bits]."""
    words = np.ascontiguousarray(weight, dtype="<u4")
    stream = np.unpackbits(words.view(np.uint8), axis=-1, bitorder="little")
    count = stream.shape[-1] // bits
    fields = stream[..., : count * bits].reshape(*stream.shape[:-1], count, bits).astype(np.int64)
    return (fields << np.arange(bits)).sum(axis=-1)


def pack(values: np.ndarray, bits: int) -> np.ndarray:
    """Integer values [..., n] (n * bits a multiple of 32) -> uint32 words."""
    values = np.asarray(values, dtype=np.int64)
    assert values.shape[-1] * bits % 32 == 0
    assert values.min(initial=0) >= 0 and values.max(initial=0) < (1 << bits)
    fields = ((values[..., None] >> np.arange(bits)) & 1).astype(np.uint8)
    stream = fields.reshape(*values.shape[:-1], values.shape[-1] * bits)
    packed = np.packbits(stream, axis=-1, bitorder="little")
    return np.ascontiguousarray(packed).view("<u4").astype(np.uint32)


def dequantize(stack: Stack) -> np.ndarray:
    """The stack's weights as float64 [..., out, in]: scale * q + bias, exactly."""
    q = unpack(stack.weight, stack.bits).astype(np.float64)
    scales = np.repeat(to_f32(stack.scales).astype(np.float64), stack.group, axis=-1)
    biases = np.repeat(to_f32(stack.biases).astype(np.float64), stack.group, axis=-1)
    return scales * q + biases


def quantize(w: np.ndarray, group: int, bits: int) -> Stack:
    """float [..., out, in] -> a Stack: per group, scale = (max - min) / (2^bits - 1) and
    bias = min (both bf16), q = round((w - bias) / scale) clipped to the width."""
    w = np.asarray(w, dtype=np.float64)
    g = w.reshape(*w.shape[:-1], w.shape[-1] // group, group)
    lo, hi = g.min(axis=-1), g.max(axis=-1)
    steps = (1 << bits) - 1
    scales = from_float(np.maximum((hi - lo) / steps, 1e-8))
    # Rounded up to the next bf16 where rounding fell short, so the steps span the group.
    short = to_f32(scales).astype(np.float64) * steps < hi - lo
    scales = (scales + short.astype(np.uint16)).astype(np.uint16)
    biases = from_float(lo)
    s = to_f32(scales).astype(np.float64)[..., None]
    b = to_f32(biases).astype(np.float64)[..., None]
    q = np.clip(np.rint((g - b) / s), 0, (1 << bits) - 1).astype(np.int64)
    return Stack(pack(q.reshape(w.shape), bits), scales, biases, group, bits)


def _slot_matrices(stack: Stack, chosen, shared: Stack | None) -> list[np.ndarray]:
    """float64 matrices, one per slot; the last is the shared leaf's when declared."""
    chosen = np.asarray(chosen, dtype=np.int64).reshape(-1)
    experts, out_features = stack.weight.shape[0], stack.weight.shape[1]
    mats = []
    for j, e in enumerate(chosen):
        if shared is not None and j == len(chosen) - 1:
            mats.append(dequantize(shared))
        elif 0 <= e < experts:
            mats.append(dequantize(Stack(stack.weight[e], stack.scales[e], stack.biases[e],
                                         stack.group, stack.bits)))
        else:
            mats.append(np.zeros((out_features, stack.in_features)))
    return mats


def sigmoid_bf16(g: np.ndarray) -> np.ndarray:
    """T(1 / (1 + exp(-g))) with each operation in fp32 (the kernels' expression)."""
    g = np.asarray(g, dtype=np.float32)
    with np.errstate(over="ignore"):
        e = np.exp(-g, dtype=np.float32)
    den = (np.float32(1.0) + e).astype(np.float32)
    return to_f32(from_float((np.float32(1.0) / den).astype(np.float32)))


def gate_up(x_bits: np.ndarray, stack: Stack, chosen, *, limit: float | None = None,
            shared: Stack | None = None) -> np.ndarray:
    """x [H] bf16 bits, stack [E, 2I, H] interleaved -> activation [slots, I] bf16 bits."""
    x = to_f32(np.asarray(x_bits).reshape(-1)).astype(np.float64)
    out = []
    for m in _slot_matrices(stack, chosen, shared):
        r = to_f32(f64_to_bf16(m @ x)).reshape(-1, 2)
        g, u = r[:, 0], r[:, 1]
        if limit is not None:
            g = np.minimum(g, np.float32(limit))
            u = np.clip(u, np.float32(-limit), np.float32(limit))
        a = to_f32(from_float(g * sigmoid_bf16(g)))
        out.append(from_float(a * u))
    return np.stack(out)


def down_combine(act_bits: np.ndarray, stack: Stack, chosen, weights,
                 residual_bits: np.ndarray | None, *, shared: Stack | None = None) -> np.ndarray:
    """act [slots, I] bf16 bits, stack [E, H, I], chosen [slots], weights [slots] fp32,
    residual [H] bf16 bits or None -> [H] bf16 bits."""
    mats = _slot_matrices(stack, chosen, shared)
    act = to_f32(np.asarray(act_bits).reshape(len(mats), -1)).astype(np.float64)
    weights = np.asarray(weights, dtype=np.float32).reshape(-1)
    acc = np.zeros(mats[0].shape[0], dtype=np.float32)
    for j, m in enumerate(mats):
        t = to_f32(f64_to_bf16(m @ act[j])).astype(np.float64)
        term = (t * np.float64(weights[j])).astype(np.float32)
        acc = (acc + to_f32(from_float(term))).astype(np.float32)
    out = to_f32(from_float(acc))
    if residual_bits is not None:
        out = (out + to_f32(np.asarray(residual_bits).reshape(-1))).astype(np.float32)
    return from_float(out)

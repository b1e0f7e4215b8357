"""Routed expert MLP of one token over NVFP4 expert stacks (TEST INFRASTRUCTURE ONLY;
see oracle/__init__.py).

Format: MLX's mode "nvfp4", the `QuantizedSwitchLinear` leaf (core/layers.py:164-197),
as core/kernels/shared/nvfp4/qmoe.py:8-50 decodes it:

- weight [E, out, in / 8] uint32: the e2m1 codes of mode "mxfp4" (two per byte, the low
  nibble first), read by oracle.mxfp4.codes;
- scales [E, out, in / 16] uint8: one e4m3 byte per 16 values, decoded as mlx decodes it:
  sign bit 7, exponent bits 6-3 (bias 7), mantissa bits 2-0; exponent 0 is subnormal
  (m / 8 * 2^-6); every other code, the all-ones 0x7F and 0xFF included, is
  (-1)^sign * 2^(e - 7) * (1 + m / 8), so 0x7F is 480 and not a NaN;
- no bias.

gate_up (core/kernels/gate_up/nvfp4.py:24-68), interleaved rows, the plain SwiGLU chain:

    r   = sum over groups of scale * sum_j x_j v_j           fp32 there; float64 here
    g   = T(r_gate), u = T(r_up)
    sig = T(1 / (1 + exp(-g)))                               each op in fp32
    y   = T(T(g * sig) * u)

down_combine (core/kernels/down_combine/nvfp4.py:16-61):

    acc = sum over slots in order of T(fp32(T(t) * w))       fp32
    y   = T(fp32(T(acc) + residual))

down_combine_shared, the packed form (core/kernels/down_combine/nvfp4_packed.py:108-138),
for each token of a batch: slot s < k runs expert chosen[s], slot k the shared stack,
unweighted; every step is bf16:

    d_s   = T(t_s)                                           t_s the exact dot here
    total = T(T(d_s * T(w_s)) + total)    s < k, in order   each op in fp32
    y     = T(residual + T(total + d_k))

halved_scales restates the halved group-32 plane and its certificate
(core/kernels/shared/nvfp4/packed.py:126-164).

An expert id outside [0, experts) contributes zero rows (the HIP kernels' guard).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .bf16 import from_float, to_f32
from .mxfp4 import E2M1, codes, pack  # noqa: F401  (pack re-exported for the tests)

GROUP = 16


def _e4m3_value(byte: int) -> float:
    sign = -1.0 if byte & 0x80 else 1.0
    e, m = (byte >> 3) & 0xF, byte & 0x7
    return sign * (m / 8 * 2.0 ** -6 if e == 0 else 2.0 ** (e - 7) * (1 + m / 8))


E4M3 = np.array([_e4m3_value(b) for b in range(256)])


@dataclass
class Stack:
    weight: np.ndarray   # uint32 [..., out, in / 8]
    scales: np.ndarray   # uint8 [..., out, in / 16]


def scale_values(scales: np.ndarray) -> np.ndarray:
    """e4m3 bytes -> float64 factors."""
    return E4M3[np.asarray(scales, dtype=np.uint8)]


def dequantize(stack: Stack) -> np.ndarray:
    """float64 [..., out, in] weights."""
    return E2M1[codes(stack.weight)] * np.repeat(scale_values(stack.scales), GROUP, axis=-1)


def _slot(stack: Stack, e: int) -> np.ndarray:
    experts, out = stack.weight.shape[0], stack.weight.shape[1]
    if not 0 <= e < experts:
        return np.zeros((out, stack.weight.shape[2] * 8))
    return dequantize(Stack(stack.weight[e], stack.scales[e]))


def _T(values) -> np.ndarray:
    return to_f32(from_float(np.asarray(values, dtype=np.float32)))


def swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """The plain chain on bf16-valued g and u, each step rounded to T -> bf16 bits."""
    with np.errstate(over="ignore"):
        e = np.exp((-g).astype(np.float32), dtype=np.float32)
    sig = _T((np.float32(1.0) / (np.float32(1.0) + e)).astype(np.float32))
    act = _T(g * sig)
    return from_float(act * u)


def gate_up(x_bits: np.ndarray, stack: Stack, chosen) -> np.ndarray:
    """x [H] bf16 bits, stack [E, 2I, ...] -> [slots, I] bf16 bits."""
    x = to_f32(np.asarray(x_bits).reshape(-1)).astype(np.float64)
    out = []
    for e in np.asarray(chosen).reshape(-1):
        r = _slot(stack, int(e)) @ x   # the kernels' fp32 sum, exact here, rounded once to T
        out.append(swiglu(_T(r[0::2].astype(np.float32)), _T(r[1::2].astype(np.float32))))
    return np.stack(out)


def down_combine(act_bits: np.ndarray, stack: Stack, chosen, weights,
                 residual_bits: np.ndarray | None) -> np.ndarray:
    """act [slots, I] bf16 bits, stack [E, H, ...], weights [slots] fp32 -> [H] bf16 bits."""
    chosen = np.asarray(chosen).reshape(-1)
    act = to_f32(np.asarray(act_bits).reshape(len(chosen), -1)).astype(np.float64)
    weights = np.asarray(weights, dtype=np.float32).reshape(-1)
    acc = np.zeros(stack.weight.shape[1], dtype=np.float32)
    for j, e in enumerate(chosen):
        if not 0 <= int(e) < stack.weight.shape[0]:
            continue
        t = _T((_slot(stack, int(e)) @ act[j]).astype(np.float32)).astype(np.float64)
        acc = (acc + _T((t * np.float64(weights[j])).astype(np.float32))).astype(np.float32)
    out = _T(acc)
    if residual_bits is not None:
        out = (out + to_f32(np.asarray(residual_bits).reshape(-1))).astype(np.float32)
    return from_float(out)


PATCH_BYTES = 128   # shared/nvfp4/packed.py:63 (SCALE_PATCH_BYTES)


def halved_scales(scales: np.ndarray, allowed_pairs=(0,)) -> np.ndarray | None:
    """packed.py:126-164 `halved_group32_scales`: the plane read as [size / 2, 2] byte
    pairs keeps each even byte behind a PATCH_BYTES header holding the odd bytes of the
    allowed pairs; None unless every other odd byte equals its even partner and every byte
    is below 128."""
    flat = np.ascontiguousarray(scales, dtype=np.uint8).reshape(-1, 2)
    allowed = list(allowed_pairs)
    mismatch = flat[:, 0] != flat[:, 1]
    mismatch[allowed] = False
    if mismatch.any() or int(np.asarray(scales).max(initial=0)) >= 128:
        return None
    header = np.zeros(PATCH_BYTES, dtype=np.uint8)
    header[: len(allowed)] = flat[allowed, 1]
    return np.concatenate([header, flat[:, 0]])


def down_combine_shared(act_bits: np.ndarray, stack: Stack, shared: Stack, chosen, weights,
                        residual_bits: np.ndarray) -> np.ndarray:
    """act [T, k + 1, I] bf16 bits (the shared slot last), stack [E, H, ...], shared
    [H, ...], chosen [T, k] (or [T, k + 1], the last ignored), weights likewise fp32,
    residual [T, H] bf16 bits -> [T, H] bf16 bits."""
    act = to_f32(np.asarray(act_bits)).astype(np.float64)
    tokens, slots = act.shape[0], act.shape[1]
    k = slots - 1
    chosen = np.asarray(chosen).reshape(tokens, -1)[:, :k]
    weights = np.asarray(weights, dtype=np.float32).reshape(tokens, -1)[:, :k]
    residual = to_f32(np.asarray(residual_bits).reshape(tokens, -1))
    shared_matrix = dequantize(shared)
    out = []
    for t in range(tokens):
        total = np.zeros(stack.weight.shape[1], dtype=np.float32)
        for s in range(k):
            d = _T((_slot(stack, int(chosen[t, s])) @ act[t, s]).astype(np.float32))
            w = _T(weights[t, s])
            total = _T(_T(d * w) + total)
        d_shared = _T((shared_matrix @ act[t, k]).astype(np.float32))
        out.append(from_float((residual[t] + _T(total + d_shared)).astype(np.float32)))
    return np.stack(out)

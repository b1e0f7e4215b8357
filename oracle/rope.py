"""Per-head q/k RMSNorm + half-split RoPE (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

Table-driven variant, restating core/kernels/qkv_rope/qk_norm_rope.py:21-24,120-140,
295-308 and the composition of tests/test_kernel_qk_norm_rope.py:95-126:

    n        = rms_norm(x, w, eps) per head          (oracle.add_norm.rms_norm rounding)
    a, b     = R(n_p * R(mscale)), R(n_{p+P} * R(mscale))          for p < P
    out_p    = R(a * cos[pos, p] - b * sin[pos, p])
    out_{p+P}= R(a * sin[pos, p] + b * cos[pos, p])
    out_d    = n_d                                                   for d >= 2P

with every product and sum in float32 (no fused multiply-add). Inputs are token-major
[T, H, D]; outputs head-major [H, T, D] (qk_norm_rope.py:163-175).

Epilogue variant (core/kernels/qkv_rope/epilogue.py:57-63): the same with the angle
derived from the position, `f32(pos) * exp2(-(i / P) * f32(log2(base)))` in float32,
with exp2, cos and sin evaluated in float64 and rounded once to float32.
"""

from __future__ import annotations

import math

import numpy as np

from .add_norm import rms_norm
from .bf16 import R, to_bf16, to_f32


def angle_table(rows: int, pairs: int, base: float, first: int = 0):
    """(cos, sin) float32 [rows, pairs] for positions first .. first+rows-1.

    The fp64 build of tests/test_kernel_qk_norm_rope.py:51-66 (`inverse =
    exp(-log(base) * i / pairs)`, `theta = pos * inverse`), rounded to float32 once.
    """
    inverse = np.exp(-np.log(base) * np.arange(pairs) / pairs)
    theta = (first + np.arange(rows))[:, None] * inverse[None, :]
    return np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)


def laguna_inverse(pairs: int, base: float) -> np.ndarray:
    """`base ** (arange(0, D, 2, fp32) / D)` of models/laguna/layers/attention.py:238-239 as
    fp32 operations, each correctly rounded (the power evaluated in float64 from the fp32
    operands and rounded once)."""
    exponents = np.arange(0, 2 * pairs, 2, dtype=np.float32) / np.float32(2 * pairs)
    return np.power(np.float64(np.float32(base)), exponents.astype(np.float64)).astype(np.float32)


def laguna_angle_table(rows: int, pairs: int, base: float | None = None, first: int = 0,
                       inverse: np.ndarray | None = None):
    """(cos, sin) float32 [rows, pairs] in the fp32 order of models/laguna/layers/
    attention.py:236-243: theta = arange(fp32) / inverse as an fp32 quotient (formed in
    float64 and rounded once), cos and sin of that fp32 angle in float64, rounded once.
    `inverse` is the YaRN table when given (used as is), else `laguna_inverse`."""
    inverse = laguna_inverse(pairs, base) if inverse is None else np.asarray(inverse, np.float32)
    positions = np.arange(first, first + rows, dtype=np.float64).astype(np.float32)
    theta = (positions.astype(np.float64)[:, None] / inverse.astype(np.float64)[None, :]).astype(np.float32)
    wide = theta.astype(np.float64)
    return np.cos(wide).astype(np.float32), np.sin(wide).astype(np.float32)


def epilogue_angles(positions: np.ndarray, pairs: int, base: float):
    """(cos, sin) float32 [len(positions), pairs] by the in-kernel derivation of
    core/kernels/qkv_rope/epilogue.py:57-63."""
    log2_base = np.float32(math.log2(base))
    d = np.arange(pairs, dtype=np.float32) / np.float32(pairs)
    exponent = (-d) * log2_base
    frequency = np.exp2(exponent.astype(np.float64)).astype(np.float32)
    angle = np.asarray(positions).astype(np.float32)[:, None] * frequency[None, :]
    wide = angle.astype(np.float64)
    return np.cos(wide).astype(np.float32), np.sin(wide).astype(np.float32)


def norm_rotate(raw, weight, cos, sin, eps: float, pairs: int, mscale: float = 1.0):
    """raw [T, H, D] bf16 bits, (cos, sin) [T, P] fp32 -> [H, T, D] bf16 bits."""
    normed = rms_norm(raw, weight, eps)  # per head: last axis is D
    n = to_f32(normed)
    scale = R(np.array([mscale], dtype=np.float32))[0]
    first = R(n[..., :pairs] * scale)
    second = R(n[..., pairs : 2 * pairs] * scale)
    c = cos[:, None, :]
    s = sin[:, None, :]
    rotated_first = to_bf16(first * c - second * s)
    rotated_second = to_bf16(first * s + second * c)
    out = np.concatenate([rotated_first, rotated_second, normed[..., 2 * pairs :]], axis=-1)
    return np.ascontiguousarray(out.transpose(1, 0, 2))


def qk_norm_rope(raw_q, raw_k, q_weight, k_weight, cos_table, sin_table, offset: int,
                 eps: float, pairs: int, mscale: float = 1.0):
    """Table rows offset .. offset+T-1 -> (q [Hq, T, D], k [Hkv, T, D]) bf16 bits."""
    length = raw_q.shape[0]
    cos = cos_table[offset : offset + length, :pairs]
    sin = sin_table[offset : offset + length, :pairs]
    return (
        norm_rotate(raw_q, q_weight, cos, sin, eps, pairs, mscale),
        norm_rotate(raw_k, k_weight, cos, sin, eps, pairs, mscale),
    )


def rope_epilogue(fused, query_heads: int, kv_heads: int, head_dim: int, q_weight,
                  k_weight, offset: int, base: float, eps: float):
    """fused [T, (Hq + 2 Hkv) * D] bf16 bits -> (q [Hq, T, D], k [Hkv, T, D])."""
    length = fused.shape[0]
    pairs = head_dim // 2
    cos, sin = epilogue_angles(offset + np.arange(length), pairs, base)
    q_width = query_heads * head_dim
    raw_q = fused[:, :q_width].reshape(length, query_heads, head_dim)
    raw_k = fused[:, q_width : q_width + kv_heads * head_dim].reshape(length, kv_heads, head_dim)
    return (
        norm_rotate(raw_q, q_weight, cos, sin, eps, pairs),
        norm_rotate(raw_k, k_weight, cos, sin, eps, pairs),
    )

"""MoE routing (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

Restates the softmax routing chain (core/kernels/route/default.py:44-69;
models/qwen3/layers/moe.py:34-42) with the definitions the build adopts:

- logits = bf16(n . W_e), the dot product evaluated in float64 and rounded once (the
  correctly rounded value; the reference leaves the fp32 accumulation order free);
- selection: the k largest bf16 logits, descending, exact ties to the LOWER expert
  index (the rule of core/kernels/route/ordinal.py:1-27; the reference's softmax chain
  breaks ties toward the higher index, default.py:7-9). Softmax is monotone, so this is
  a stable descending sort of the probabilities;
- weights: p = softmax(logits) in float32, w = p[sel] / sum(p[sel]) in float32.

The fused residual router (core/kernels/route/residual.py:117-299) is the residual
join of oracle/add_norm.py followed by the above.
"""

from __future__ import annotations

import numpy as np

from .activations import f64_to_bf16
from .add_norm import add_rms_norm
from .bf16 import to_f32


def router_logits(n_bits: np.ndarray, w_bits: np.ndarray) -> np.ndarray:
    """[T, H] x [E, H]^T in float64, rounded once to bf16 bits [T, E]."""
    return f64_to_bf16(to_f32(n_bits).astype(np.float64) @ to_f32(w_bits).astype(np.float64).T)


def order_keys(logit_bits: np.ndarray) -> np.ndarray:
    """Order-preserving integer map of bf16 bits: -0 folded onto +0, NaN above all."""
    b = np.asarray(logit_bits, dtype=np.uint16).astype(np.int64)
    b = np.where(b == 0x8000, 0, b)
    key = np.where(b & 0x8000, (~b) & 0xFFFF, b | 0x8000)
    return np.where((b & 0x7FFF) > 0x7F80, 0xFFFF, key)


def select(logit_bits: np.ndarray, k: int) -> np.ndarray:
    """Top-k expert indices per row, descending, lowest index first on ties."""
    keys = order_keys(logit_bits)
    # Stable ascending argsort of -key keeps equal keys in ascending index order.
    return np.argsort(-keys, axis=-1, kind="stable")[..., :k].astype(np.int32)


def renormalised_weights(logit_bits: np.ndarray, indices: np.ndarray) -> np.ndarray:
    logits = to_f32(logit_bits)
    shifted = logits - logits.max(axis=-1, keepdims=True)
    e = np.exp(shifted, dtype=np.float32)
    p = (e / e.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    kept = np.take_along_axis(p, indices.astype(np.int64), axis=-1)
    return (kept / kept.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)


def softmax_topk(logit_bits: np.ndarray, k: int):
    indices = select(logit_bits, k)
    return indices, renormalised_weights(logit_bits, indices)


def residual_rms_router(x_bits, branch_bits, norm_bits, router_bits, eps: float, k: int):
    """(summed, normalized, logits, indices, weights)."""
    summed, normalized = add_rms_norm(x_bits, branch_bits, norm_bits, eps)
    logits = router_logits(normalized, router_bits)
    indices, weights = softmax_topk(logits, k)
    return summed, normalized, logits, indices, weights

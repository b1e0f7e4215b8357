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

Sigmoid routing with a correction bias (core/kernels/route/ordinal.py:200-286,
`router_tournament` / `OrdinalRoute`; the keys of route/residual.py:109-115):

- score = sigmoid(x) of the float32 logit, the stable form of ordinal.py:74-76
  (y = 1 / (1 + exp|x|), x < 0 ? y : 1 - y) evaluated in float64 and rounded once to
  float32 (the correctly rounded value; the reference's Metal `exp` is not);
- key = ordinal(-(score + bias)), the sum in float32, `ordinal` the map of
  ordinal.py:37-47 (ascending unsigned order = ascending float order, +-0 one value,
  NaN above everything);
- selection: the first k of the stable ascending order of the keys (descending
  score + bias, lower index first on ties, NaN last);
- weights: the winners' unbiased scores over their float32 sum, taken in winner order
  (ordinal.py:183-193), divided in float32.

NaN in the softmax chain ranks last as well, the place ordinal.py gives a NaN score.

The two other softmax declarations of the reference's `Route` (`softmax_topk_slots`):

- `normalize=False` (core/kernels/route/default.py:61-63 skips the division;
  models/qwen3/layers/moe.py:50-52 declares `normalize=norm_topk`): the weights are
  the kept float32 probabilities themselves, p[sel];
- `shared=True` (core/kernels/route/softmax_topk.py:67-72 and default.py:65-68;
  models/qwen3_5/layers/moe.py:157-162): the row carries one more logit after the
  routed experts, the shared expert's gate; the selection runs over the routed logits
  only, and one more slot follows the k routed ones: index `experts`, weight the
  float32 sigmoid of that logit (the kernel's stable form, `sigmoid_f32` below,
  correctly rounded; the reference rounds it to the logits' dtype, bf16).
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
    """Order-preserving integer map of bf16 bits: -0 folded onto +0, NaN below all (so a
    NaN logit ranks last, as ordinal.py:37-47 ranks a NaN score)."""
    b = np.asarray(logit_bits, dtype=np.uint16).astype(np.int64)
    b = np.where(b == 0x8000, 0, b)
    key = np.where(b & 0x8000, (~b) & 0xFFFF, b | 0x8000)
    return np.where((b & 0x7FFF) > 0x7F80, 0, key)


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


def softmax_probabilities(logit_bits: np.ndarray) -> np.ndarray:
    """softmax of the bf16 logits over the row, in float32 (default.py:46)."""
    logits = to_f32(logit_bits)
    shifted = logits - logits.max(axis=-1, keepdims=True)
    e = np.exp(shifted, dtype=np.float32)
    return (e / e.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)


def softmax_topk_slots(logit_bits: np.ndarray, k: int, *, normalize: bool = True,
                       shared: bool = False):
    """(indices [..., k + shared] int32, weights fp32) of the softmax declaration with
    or without renormalisation and with or without the shared slot (default.py:44-69,
    softmax_topk.py:20-75)."""
    logit_bits = np.asarray(logit_bits, dtype=np.uint16)
    experts = logit_bits.shape[-1] - (1 if shared else 0)
    routed = logit_bits[..., :experts]
    indices = select(routed, k)
    if normalize:
        weights = renormalised_weights(routed, indices)
    else:
        weights = np.take_along_axis(softmax_probabilities(routed), indices.astype(np.int64), axis=-1)
    if shared:
        slot = np.full((*indices.shape[:-1], 1), experts, dtype=np.int32)
        gate = sigmoid_f32(to_f32(logit_bits[..., experts:]))
        indices = np.concatenate([indices, slot], axis=-1)
        weights = np.concatenate([weights, gate.astype(np.float32)], axis=-1)
    return indices, weights.astype(np.float32)


def residual_rms_router(x_bits, branch_bits, norm_bits, router_bits, eps: float, k: int):
    """(summed, normalized, logits, indices, weights)."""
    summed, normalized = add_rms_norm(x_bits, branch_bits, norm_bits, eps)
    logits = router_logits(normalized, router_bits)
    indices, weights = softmax_topk(logits, k)
    return summed, normalized, logits, indices, weights


def sigmoid_f32(x: np.ndarray) -> np.ndarray:
    """Correctly rounded float32 sigmoid of float32 values (ordinal.py:74-76's stable
    form, in float64, rounded once)."""
    x64 = np.asarray(x, dtype=np.float32).astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        y = 1.0 / (1.0 + np.exp(np.abs(x64)))
        score = np.where(x64 < 0.0, y, 1.0 - y)
    return score.astype(np.float32)


def ordinal(key: np.ndarray) -> np.ndarray:
    """ordinal.py:37-47 `router_key_ordinal`: uint32 whose ascending order is the float
    order of `key` (float32), +-0 -> 0x80000000, NaN -> 0xFFFFFFFF."""
    bits = np.ascontiguousarray(key, dtype=np.float32).view(np.uint32).astype(np.uint64)
    magnitude = bits & 0x7FFFFFFF
    out = np.where(bits & 0x80000000, (~bits) & 0xFFFFFFFF, bits ^ 0x80000000)
    out = np.where(magnitude == 0, 0x80000000, out)
    out = np.where(magnitude > 0x7F800000, 0xFFFFFFFF, out)
    return out.astype(np.uint32)


def sigmoid_keys(logits_f32: np.ndarray, bias: np.ndarray):
    """(scores, keys) of a row of float32 logits: scores = sigmoid_f32(logits),
    keys = ordinal(-(score + bias)) with the sum rounded to float32 (ordinal.py:74-78,
    residual.py:109-115)."""
    scores = sigmoid_f32(logits_f32)
    with np.errstate(invalid="ignore"):
        biased = (scores + np.asarray(bias, dtype=np.float32)).astype(np.float32)
    return scores, ordinal(-biased)


def ordinal_select(keys: np.ndarray, k: int) -> np.ndarray:
    """The first k of the stable ascending order of the keys (ties: lower index)."""
    return np.argsort(keys, axis=-1, kind="stable")[..., :k].astype(np.int32)


def ordinal_weights(scores: np.ndarray, indices: np.ndarray) -> np.ndarray:
    """ordinal.py:183-193: the winners' unbiased scores over their float32 sum, the sum
    taken in winner order, the quotient rounded to float32."""
    picked = np.take_along_axis(scores, indices.astype(np.int64), axis=-1).astype(np.float32)
    total = np.zeros(picked.shape[:-1], dtype=np.float32)
    for j in range(picked.shape[-1]):
        total = (picked[..., j] + total).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        return (picked / total[..., None]).astype(np.float32)


def sigmoid_topk(logits_f32: np.ndarray, bias: np.ndarray, k: int):
    """(indices, weights, keys) of sigmoid routing with a correction bias
    (ordinal.py:200-286, `router_tournament`)."""
    scores, keys = sigmoid_keys(logits_f32, bias)
    indices = ordinal_select(keys, k)
    return indices, ordinal_weights(scores, indices), keys


def residual_rms_router_sigmoid(x_bits, branch_bits, norm_bits, router_bits, bias,
                                eps: float, k: int):
    """The fused router's sigmoid form (residual.py:117-299): (summed, normalized,
    logits, keys, indices, weights), the keys built from the bf16 logits."""
    summed, normalized = add_rms_norm(x_bits, branch_bits, norm_bits, eps)
    logits = router_logits(normalized, router_bits)
    indices, weights, keys = sigmoid_topk(to_f32(logits), bias, k)
    return summed, normalized, logits, keys, indices, weights

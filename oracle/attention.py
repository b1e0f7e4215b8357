"""One decode step of an attention layer over a KV cache (TEST INFRASTRUCTURE ONLY; see
oracle/__init__.py).

Restates the fused steps core/kernels/attention/full.py:133-471 (a fixed cache) and
sliding.py:136-430 (a ring), whose Core chain is core/kernels/attention/default.py:
114-156 (rms_norm, rope, `cache.update_and_fetch`, scaled_dot_product_attention):

- the new query and key rows: per-head RMSNorm and the half-split rotation with the
  folded mscale, exactly as oracle.rope.norm_rotate (the fused kernels' rounding points,
  full.py:175-209), cos || sin from the angle row of the step's position;
- the cache write (core/cache/kv.py:131-170, 326-381): a fixed cache writes row p and
  attends rows [0, p]; a ring of `window` rows writes row p % window and attends rows
  [0, min(p + 1, window));
- attention: s_r = scale * q . k_r, softmax over the attended rows, o = sum_r p_r v_r,
  evaluated in float64 and rounded once to bf16 (the kernels keep fp32 with an online
  softmax; their order is free). Query head h reads kv head h // (heads / kv_heads)
  (full.py:146-149).

`sink_attend` restates the attention of a layer with learned sink logits
(core/kernels/attention/sink.py:60-166): the roped query against the cached rows, the
sink in the softmax's denominator only, a boolean band or an additive mask.
"""

from __future__ import annotations

import numpy as np

from .activations import f64_to_bf16
from .bf16 import to_f32
from .rope import norm_rotate

HEAD_DIM = 128


def step_rows(position: int, capacity: int, window: int) -> tuple[int, int]:
    """(write row, attended row count) for a fixed cache (window 0) or a ring."""
    if window:
        return position % window, min(position + 1, window)
    return position, min(position + 1, capacity)


def roped(raw_bits: np.ndarray, weight_bits: np.ndarray, angle_row: np.ndarray, eps: float,
          pairs: int, mscale: float) -> np.ndarray:
    """[heads * 128] raw rows -> [heads, 128] normed and rotated bf16 bits."""
    raw = np.asarray(raw_bits).reshape(1, -1, HEAD_DIM)
    cos = np.asarray(angle_row[:pairs], dtype=np.float32)[None]
    sin = np.asarray(angle_row[pairs : 2 * pairs], dtype=np.float32)[None]
    return norm_rotate(raw, weight_bits, cos, sin, eps, pairs, mscale)[:, 0]


def attend(q_bits: np.ndarray, k_rows: np.ndarray, v_rows: np.ndarray, scale: float) -> np.ndarray:
    """q [heads, 128], k/v [kv_heads, rows, 128] bf16 bits -> [heads, 128] bf16 bits."""
    heads, kv_heads = q_bits.shape[0], k_rows.shape[0]
    gqa = heads // kv_heads
    q = to_f32(q_bits).astype(np.float64)
    k = to_f32(k_rows).astype(np.float64)
    v = to_f32(v_rows).astype(np.float64)
    out = np.empty((heads, HEAD_DIM), dtype=np.float64)
    for h in range(heads):
        s = float(scale) * (k[h // gqa] @ q[h])
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v[h // gqa]
    return f64_to_bf16(out)


def decode_step(raw_q, raw_k, raw_v, q_weight, k_weight, angle_row, k_cache, v_cache,
                position: int, *, window: int, scale: float, eps: float, pairs: int,
                mscale: float = 1.0):
    """Returns (context [heads, 128], new key cache, new value cache), all bf16 bits.
    Caches are [kv_heads, capacity, 128]; the inputs are not modified."""
    kv_heads, capacity, _ = k_cache.shape
    write, count = step_rows(position, capacity, window)
    q = roped(raw_q, q_weight, angle_row, eps, pairs, mscale)
    k = roped(raw_k, k_weight, angle_row, eps, pairs, mscale)
    keys, values = k_cache.copy(), v_cache.copy()
    keys[:, write] = k
    values[:, write] = np.asarray(raw_v).reshape(kv_heads, HEAD_DIM)
    return attend(q, keys[:, :count], values[:, :count], scale), keys, values


def sink_attend(q_bits: np.ndarray, k_rows: np.ndarray, v_rows: np.ndarray, sink_bits: np.ndarray,
                mask, scale: float) -> np.ndarray:
    """core/kernels/attention/sink.py:60-166 (`sink_attention`): q [heads, D], k/v
    [kv_heads, rows, D] bf16 bits, sinks [heads] bf16 bits, mask None (every row), a
    boolean band [rows] (True attends) or an additive float [rows] whose infinite entries
    drop the row -> [heads, D] bf16 bits. In float64, rounded once to bf16:

        s_r = scale * q . k_r + mask_r,  M = max(sink, max_r s_r)
        o   = sum_r exp(s_r - M) v_r / (exp(sink - M) + sum_r exp(s_r - M))
    """
    heads, kv_heads, rows = q_bits.shape[0], k_rows.shape[0], k_rows.shape[1]
    gqa = heads // kv_heads
    if mask is None:
        additive = np.zeros(rows)
    else:
        flat = np.asarray(mask).reshape(-1)
        additive = np.where(flat, 0.0, -np.inf) if flat.dtype == np.bool_ else flat.astype(np.float64)
    keep = ~np.isinf(additive)
    q = to_f32(q_bits).astype(np.float64)
    k = to_f32(k_rows).astype(np.float64)
    v = to_f32(v_rows).astype(np.float64)
    sinks = to_f32(np.asarray(sink_bits).reshape(-1)).astype(np.float64)
    out = np.empty(q.shape, dtype=np.float64)
    for h in range(heads):
        s = (float(scale) * (k[h // gqa] @ q[h]) + additive)[keep]
        top = max(sinks[h], s.max()) if s.size else sinks[h]
        p = np.exp(s - top)
        out[h] = (p @ v[h // gqa][keep]) / (np.exp(sinks[h] - top) + p.sum())
    return f64_to_bf16(out)

"""HIP bindings of the qkv prologue: the table-driven norm+rotary and the rope epilogue.

`HipQkNormRope` serves the declarations core/kernels/qkv_rope/qk_norm_rope.py:611-651
(`QkNormRope.build`) serves: `angles` + `rotary_pairs` + both norms, partial rotary and
the mscale pre-scale included, for any segment length. `HipRopeEpilogue` serves
core/kernels/qkv_rope/epilogue.py:157-195 (`RopeEpilogue.build`): a bare `base`, full
rotary, no mscale, now for any number of tokens rather than one. Both read q and k
straight out of the fused projection rows (no split copy) and write head-major q, k;
v stays a view of the projection. A segment the kernels do not serve (batch > 1, a
tensor offset) goes to the Core fallback, as in the reference, and the hand-off is
recorded (`resolve.record_fallback`).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from ...runtime import ops
from ..resolve import record_fallback
from .._device import hip_device
from .default import DefaultQkvRope
from .atlas import AngleAtlas
from .kernel import AngleTable, Angles, Projection, QkvRopeStrategy

HEAD_DIMS = (64, 128, 256)


def qk_norm_rope_applies(head_dim: int, rotary_pairs: int) -> bool:
    """A head is head_dim/8 lanes of one 16-byte vector each; the rotary partner of
    element p (p + rotary_pairs) sits on lane `lane ^ rotary_pairs/8`, so rotary_pairs is
    8 times a power of two, and the rotary section fits in the head."""
    if head_dim not in HEAD_DIMS or rotary_pairs < 8 or rotary_pairs % 8:
        return False
    lanes = rotary_pairs // 8
    return lanes & (lanes - 1) == 0 and 2 * rotary_pairs <= head_dim


def rope_epilogue_applies(head_dim: int) -> bool:
    return qk_norm_rope_applies(head_dim, head_dim // 2)


def _fallback(projection, heads, kv_heads, head_dim, rope, eps, q_norm, k_norm):
    return DefaultQkvRope(projection, heads, kv_heads, head_dim, rope, eps, q_norm, k_norm)


def _values(fused: torch.Tensor, heads: int, kv_heads: int, head_dim: int) -> torch.Tensor:
    start = (heads + kv_heads) * head_dim
    v = fused[..., start : start + kv_heads * head_dim]
    return v.reshape(fused.shape[0], fused.shape[1], kv_heads, head_dim).transpose(1, 2)


@dataclass(frozen=True)
class HipQkNormRope(QkvRopeStrategy):
    projection: Projection
    heads: int
    kv_heads: int
    head_dim: int
    rotary_pairs: int
    eps: float
    mscale: float
    angles: Angles
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    fallback: DefaultQkvRope

    @classmethod
    def build(cls, projection, *, heads, kv_heads, head_dim, rope, eps, q_norm, k_norm,
              base, angles, rotary_pairs, mscale) -> "HipQkNormRope | None":
        if angles is None or rotary_pairs is None or q_norm is None or k_norm is None:
            return None
        if not qk_norm_rope_applies(head_dim, rotary_pairs):
            return None
        if q_norm.dtype != torch.bfloat16 or k_norm.dtype != torch.bfloat16:
            return None
        if not hip_device(q_norm, k_norm):
            return None
        return cls(projection, heads, kv_heads, head_dim, rotary_pairs, float(eps),
                   float(mscale), angles, q_norm.contiguous(), k_norm.contiguous(),
                   _fallback(projection, heads, kv_heads, head_dim, rope, eps, q_norm, k_norm))

    def _tables(self, offset: int, length: int):
        if isinstance(self.angles, AngleAtlas):
            self.angles.ensure(offset + length - 1)
            table = self.angles.table()
            return table.cos, table.sin, offset
        if isinstance(self.angles, AngleTable):
            return self.angles.cos, self.angles.sin, offset
        rows = self.angles(offset, length).to(torch.float32)
        return rows[:, : self.rotary_pairs], rows[:, self.rotary_pairs :], 0

    def __call__(self, x: torch.Tensor, offset):
        fused = self.projection(x)
        if fused.shape[0] != 1 or not isinstance(offset, int) or fused.dtype != torch.bfloat16:
            record_fallback(self, self.fallback)
            return self.fallback.epilogue(fused, offset)
        rows = fused[0]
        if rows.stride(-1) != 1:
            rows = rows.contiguous()
        q_width, kv_width = self.heads * self.head_dim, self.kv_heads * self.head_dim
        raw_q = rows[:, :q_width].unflatten(-1, (self.heads, self.head_dim))
        raw_k = rows[:, q_width : q_width + kv_width].unflatten(-1, (self.kv_heads, self.head_dim))
        cos, sin, table_offset = self._tables(offset, rows.shape[0])
        q, k = ops.qk_norm_rope(
            raw_q, raw_k, self.q_norm, self.k_norm, cos, sin, offset=table_offset,
            eps=self.eps, rotary_pairs=self.rotary_pairs, mscale=self.mscale,
        )
        return q.unsqueeze(0), k.unsqueeze(0), _values(fused, self.heads, self.kv_heads, self.head_dim)


@dataclass(frozen=True)
class HipRopeEpilogue(QkvRopeStrategy):
    projection: Projection
    heads: int
    kv_heads: int
    head_dim: int
    base: float
    eps: float
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    fallback: DefaultQkvRope

    @classmethod
    def build(cls, projection, *, heads, kv_heads, head_dim, rope, eps, q_norm, k_norm,
              base, angles, rotary_pairs, mscale) -> "HipRopeEpilogue | None":
        if base is None or q_norm is None or k_norm is None:
            return None
        # The kernel derives a full, unscaled rotation from `base` alone
        # (core/kernels/qkv_rope/epilogue.py:176-183).
        if angles is not None or mscale != 1.0:
            return None
        if rotary_pairs is not None and 2 * rotary_pairs != head_dim:
            return None
        if not rope_epilogue_applies(head_dim):
            return None
        if q_norm.dtype != torch.bfloat16 or k_norm.dtype != torch.bfloat16:
            return None
        if not hip_device(q_norm, k_norm):
            return None
        return cls(projection, heads, kv_heads, head_dim, float(base), float(eps),
                   q_norm.contiguous(), k_norm.contiguous(),
                   _fallback(projection, heads, kv_heads, head_dim, rope, eps, q_norm, k_norm))

    def __call__(self, x: torch.Tensor, offset):
        fused = self.projection(x)
        if fused.shape[0] != 1 or not isinstance(offset, int) or fused.dtype != torch.bfloat16:
            record_fallback(self, self.fallback)
            return self.fallback.epilogue(fused, offset)
        rows = fused[0]
        if rows.stride(-1) != 1 or (rows.shape[0] > 1 and rows.stride(0) % 8):
            rows = rows.contiguous()
        q, k = ops.rope_epilogue(
            rows, self.q_norm, self.k_norm, query_heads=self.heads, kv_heads=self.kv_heads,
            head_dim=self.head_dim, offset=offset, log2_base=math.log2(self.base), eps=self.eps,
        )
        return q.unsqueeze(0), k.unsqueeze(0), _values(fused, self.heads, self.kv_heads, self.head_dim)

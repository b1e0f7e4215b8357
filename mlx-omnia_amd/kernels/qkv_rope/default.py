"""The Core qkv prologue: projection, split into head-major q/k/v, per-head RMSNorm and
the declared rotation, in torch ops.

Restates core/kernels/qkv_rope/default.py:28-89 (`split_heads`, `DefaultQkvRope`). The
rotation is the model's own `rope(x, offset)` callable; `rope_core` below is the
half-split rotation with the angle formula of mx.fast.rope that the reference's epilogue
copies (core/kernels/qkv_rope/epilogue.py:13-15,57-63), for declarations that carry a
`base`. `build` accepts every declaration, so this strategy registers last.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from ..add_norm.default import rms_norm_core
from .kernel import Projection, QkvRopeStrategy, Rotation


def split_heads(fused: torch.Tensor, *, heads: int, kv_heads: int, head_dim: int):
    """[B, L, (H + 2 Hkv) * D] -> head-major q, k, v views (default.py:28-40)."""
    batch, length = fused.shape[0], fused.shape[1]
    q_width, kv_width = heads * head_dim, kv_heads * head_dim
    q, k, v = torch.split(fused, [q_width, kv_width, kv_width], dim=-1)
    return tuple(
        part.reshape(batch, length, count, head_dim).transpose(1, 2)
        for part, count in ((q, heads), (k, kv_heads), (v, kv_heads))
    )


def rope_core(x: torch.Tensor, offset: int, *, base: float, dims: int | None = None) -> torch.Tensor:
    """Half-split (non-traditional) rotary over the first `dims` of the last axis of a
    [..., L, D] tensor at positions offset .. offset+L-1, computed in fp32 and rounded
    once to x's dtype."""
    head_dim = x.shape[-1]
    dims = head_dim if dims is None else dims
    pairs = dims // 2
    length = x.shape[-2]
    d = torch.arange(pairs, dtype=torch.float32, device=x.device) / pairs
    frequency = torch.exp2((-d * torch.tensor(math.log2(base), dtype=torch.float32)).double()).float()
    positions = torch.arange(offset, offset + length, device=x.device, dtype=torch.float32)
    angle = (positions[:, None] * frequency[None, :]).double()
    cos, sin = torch.cos(angle).float(), torch.sin(angle).float()
    wide = x.float()
    first, second = wide[..., :pairs], wide[..., pairs:dims]
    rotated = torch.cat([first * cos - second * sin, first * sin + second * cos], dim=-1)
    return torch.cat([rotated.to(x.dtype), x[..., dims:]], dim=-1)


@dataclass(frozen=True)
class DefaultQkvRope(QkvRopeStrategy):
    projection: Projection
    heads: int
    kv_heads: int
    head_dim: int
    rope: Rotation
    eps: float
    q_norm: torch.Tensor | None
    k_norm: torch.Tensor | None

    @classmethod
    def build(cls, projection, *, heads, kv_heads, head_dim, rope, eps, q_norm, k_norm,
              base, angles, rotary_pairs, mscale) -> "DefaultQkvRope":
        return cls(projection, heads, kv_heads, head_dim, rope, eps, q_norm, k_norm)

    def epilogue(self, fused: torch.Tensor, offset: int):
        """The norm and the rotation over an already projected segment."""
        q, k, v = split_heads(fused, heads=self.heads, kv_heads=self.kv_heads,
                              head_dim=self.head_dim)
        if self.q_norm is not None and self.k_norm is not None:
            q = rms_norm_core(q, self.q_norm, self.eps)
            k = rms_norm_core(k, self.k_norm, self.eps)
        return self.rope(q, offset), self.rope(k, offset), v

    def __call__(self, x: torch.Tensor, offset: int):
        return self.epilogue(self.projection(x), offset)

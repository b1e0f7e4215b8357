"""The qkv prologue: per-head q/k RMSNorm + RoPE, one facade, three bindings.

Mirrors core/kernels/qkv_rope/__init__.py:51-100. `angles` + `rotary_pairs` select the
table-driven `HipQkNormRope`; a bare `base` selects the in-kernel-angle
`HipRopeEpilogue`; everything else (and every non-gfx950 declaration) takes the Core
chain `DefaultQkvRope`, which makes the facade total.
"""

from __future__ import annotations

import torch

from ..resolve import resolve
from .atlas import AngleAtlas, rope_frequencies
from .default import DefaultQkvRope, rope_core, split_heads
from .hip import HipQkNormRope, HipRopeEpilogue, qk_norm_rope_applies, rope_epilogue_applies
from .kernel import AngleTable, Angles, Projection, QkvRopeStrategy, Rotation

__all__ = ["AngleAtlas", "rope_frequencies", 
    "AngleTable",
    "Angles",
    "DefaultQkvRope",
    "HipQkNormRope",
    "HipRopeEpilogue",
    "Projection",
    "QkvRope",
    "QkvRopeStrategy",
    "Rotation",
    "qk_norm_rope_applies",
    "rope_core",
    "rope_epilogue_applies",
    "split_heads",
]

# Tried left to right: the table-driven kernel, then the in-kernel-angle kernel; the
# Core chain at the end takes any declaration.
_STRATEGIES = (HipQkNormRope, HipRopeEpilogue, DefaultQkvRope)


class QkvRope(QkvRopeStrategy):
    """The prologue a block declares: picks its binding once, then forwards every call."""

    def __init__(
        self,
        projection: Projection,
        *,
        heads: int,
        kv_heads: int,
        head_dim: int,
        rope: Rotation,
        eps: float,
        q_norm: torch.Tensor | None = None,
        k_norm: torch.Tensor | None = None,
        base: float | None = None,
        angles: Angles | None = None,
        rotary_pairs: int | None = None,
        mscale: float = 1.0,
        reference: bool = False,
    ) -> None:
        self.strategy: QkvRopeStrategy = resolve(
            (DefaultQkvRope,) if reference else _STRATEGIES,
            projection,
            heads=heads,
            kv_heads=kv_heads,
            head_dim=head_dim,
            rope=rope,
            eps=eps,
            q_norm=q_norm,
            k_norm=k_norm,
            base=base,
            angles=angles,
            rotary_pairs=rotary_pairs,
            mscale=mscale,
        )

    def __call__(self, x: torch.Tensor, offset: int):
        return self.strategy(x, offset)

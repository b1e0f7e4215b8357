"""The embed primitive: embedding gather + RoPE atlas rows, one facade, two bindings.

Mirrors core/kernels/embed/__init__.py:30-53: `HipEmbed` serves a bf16 embedding with
fp32 atlases on a gfx950 device; `DefaultEmbed` (three gathers) serves everything else.
Both are pure copies and agree bit for bit.
"""

from __future__ import annotations

import torch

from ..resolve import resolve
from .default import DefaultEmbed
from .hip import HipEmbed, applies
from .kernel import EmbedStrategy

__all__ = ["DefaultEmbed", "Embed", "EmbedStrategy", "HipEmbed", "applies"]

_STRATEGIES = (HipEmbed, DefaultEmbed)


class Embed(EmbedStrategy):
    """The token and atlas gather a model declares: picks its binding once, then forwards."""

    def __init__(self, embedding: torch.Tensor, *, full_atlas: torch.Tensor,
                 sliding_atlas: torch.Tensor, reference: bool = False) -> None:
        self.strategy: EmbedStrategy = resolve(
            (DefaultEmbed,) if reference else _STRATEGIES,
            embedding, full_atlas=full_atlas, sliding_atlas=sliding_atlas,
        )

    def __call__(self, tokens: torch.Tensor, position: int):
        return self.strategy(tokens, position)

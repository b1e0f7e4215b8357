"""The qkv prologue's contract (core/kernels/qkv_rope/kernel.py:23-35).

`(x [batch, length, hidden], offset) -> (q [batch, heads, length, head_dim],
k [batch, kv_heads, length, head_dim], v [batch, kv_heads, length, head_dim])`: the
concatenated q/k/v projection, the per-head q/k RMSNorm, and the rotary. The declaration
splits what produces the fused tensor (`projection`) from what rotates it (`rope` in
ops, `base` for the in-kernel angle derivation, `angles` for the table-driven one).
"""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass
from typing import Protocol, runtime_checkable

import torch

Projection = Callable[[torch.Tensor], torch.Tensor]
Rotation = Callable[[torch.Tensor, int], torch.Tensor]
Angles = Callable[[int, int], torch.Tensor]


@dataclass(frozen=True)
class AngleTable:
    """A precomputed rotary table as two fp32 [positions, rotary_pairs] views.

    Calling it is the reference's `Angles` contract (core/kernels/qkv_rope/kernel.py:27):
    `(offset, length) -> [length, 2 * rotary_pairs]` rows, cosines then sines. The HIP
    strategy reads `cos`/`sin` in place instead, indexing row `offset + t` itself, so a
    separate-table layout and the reference's cos||sin atlas (`from_atlas`) both serve
    without a copy.
    """

    cos: torch.Tensor
    sin: torch.Tensor

    @classmethod
    def from_atlas(cls, atlas: torch.Tensor) -> "AngleTable":
        pairs = atlas.shape[-1] // 2
        return cls(atlas[:, :pairs], atlas[:, pairs:])

    @property
    def pairs(self) -> int:
        return self.cos.shape[-1]

    def __call__(self, offset: int, length: int) -> torch.Tensor:
        rows = slice(offset, offset + length)
        return torch.cat([self.cos[rows], self.sin[rows]], dim=-1)


@runtime_checkable
class QkvRopeStrategy(Protocol):
    def __call__(
        self, x: torch.Tensor, offset: int
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]: ...

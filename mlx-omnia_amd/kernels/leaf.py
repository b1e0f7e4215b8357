"""A norm leaf: the declaration object the residual-join facades read.

The reference's blocks hand `nn.RMSNorm` leaves (`.weight`, `.eps`) to their facades;
torch's `nn.RMSNorm` works here too, and this dataclass is the minimal stand-in.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class RMSNormLeaf:
    weight: torch.Tensor
    eps: float = 1e-6


@dataclass
class SwitchLinearLeaf:
    """A stack of expert matrices, one per row: weight [experts, out, in], the layout of
    the reference's `SwitchLinear` leaf (core/layers.py:140-154)."""

    weight: torch.Tensor

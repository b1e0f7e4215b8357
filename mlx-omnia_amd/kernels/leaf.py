"""Leaves: the declaration objects the facades read.

The reference's blocks hand `nn.RMSNorm` leaves (`.weight`, `.eps`) to the residual-join
facades, `SwitchLinear` stacks to the routed expert facades and `SwiGLU` modules to the
dense MLP facade; these are the minimal torch stand-ins.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

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


def swish(x: torch.Tensor) -> torch.Tensor:
    return x * torch.sigmoid(x)


class SwiGLU(torch.nn.Module):
    """gate||up concatenated on the output axis (gate rows first) and split back by slice,
    then the down projection: core/layers.py:253-272. The projections are bias-free
    `nn.Linear` layers, as there; `activation` is the only thing architectures vary."""

    def __init__(self, hidden: int, inner: int,
                 activation: Callable[[torch.Tensor], torch.Tensor] = swish) -> None:
        super().__init__()
        self.inner = inner
        self.gate_up_proj = torch.nn.Linear(hidden, 2 * inner, bias=False)
        self.down_proj = torch.nn.Linear(inner, hidden, bias=False)
        self._activation = activation

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gate, up = torch.split(self.gate_up_proj(x), [self.inner, self.inner], dim=-1)
        return self.down_proj(self._activation(gate) * up)

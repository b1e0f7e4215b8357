"""The Core gate/up activation: the op chain in torch, each op rounding to the input
dtype as the reference's bf16 ops do (core/layers.py:249-250 `swish`,
core/kernels/gate_up/default.py:71-81 including the swiglu_oai clamp)."""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .kernel import Activation, GateUpActivationStrategy, Layout, split


def swiglu_core(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    sigmoid = torch.sigmoid(gate.float()).to(gate.dtype)
    return (gate * sigmoid) * up


@dataclass(frozen=True)
class DefaultGateUpActivation(GateUpActivationStrategy):
    activation: Activation
    layout: Layout
    limit: float | None

    @classmethod
    def build(cls, *, activation, layout, limit) -> "DefaultGateUpActivation":
        return cls(activation, layout, limit)

    def __call__(self, gate_up: torch.Tensor, up: torch.Tensor | None = None) -> torch.Tensor:
        gate, up = split(gate_up, up, self.layout)
        if self.activation == "swiglu_oai":
            assert self.limit is not None
            gate = torch.clamp(gate, max=self.limit)
            up = torch.clamp(up, -self.limit, self.limit)
            glu = (gate * torch.sigmoid((1.702 * gate.float())).to(gate.dtype))
            return glu * (up + 1)
        if self.limit is not None:
            gate = torch.clamp(gate, max=self.limit)
            up = torch.clamp(up, -self.limit, self.limit)
        return swiglu_core(gate, up)

"""Gate/up: the activation facade (`GateUpActivation`: `HipSwiGLU` ahead of the Core
chain `DefaultGateUpActivation`) and the routed projection of a one-token step
(`GateUp` in routed.py: `HipNvfp4GateUp`, `HipMxfp4GateUp`, `HipAffineGateUp` and
`HipDenseGateUp` ahead of `DefaultGateUp`), each resolved by its declaration with the reference's
first-build-wins rule."""

from __future__ import annotations

import torch

from ..resolve import resolve
from .default import DefaultGateUpActivation, swiglu_core
from .hip import HipSwiGLU, applies
from .kernel import Activation, GateUpActivationStrategy, Layout, split
from .routed import (DefaultGateUp, GateUp, GateUpStrategy, HipAffineGateUp, HipDenseGateUp,
                     HipMxfp4GateUp, HipNvfp4GateUp, OrdinalRouting, affine_gate_up_applies,
                     dense_gate_up_applies, mxfp4_applies)

__all__ = [
    "DefaultGateUp",
    "DefaultGateUpActivation",
    "GateUp",
    "GateUpStrategy",
    "HipAffineGateUp",
    "HipDenseGateUp",
    "HipMxfp4GateUp",
    "HipNvfp4GateUp",
    "OrdinalRouting",
    "affine_gate_up_applies",
    "dense_gate_up_applies",
    "mxfp4_applies",
    "GateUpActivation",
    "GateUpActivationStrategy",
    "HipSwiGLU",
    "applies",
    "split",
    "swiglu_core",
]

_STRATEGIES = (HipSwiGLU, DefaultGateUpActivation)


class GateUpActivation(GateUpActivationStrategy):
    def __init__(self, *, activation: Activation = "swiglu", layout: Layout = "blocked",
                 limit: float | None = None, reference: bool = False) -> None:
        self.strategy: GateUpActivationStrategy = resolve(
            (DefaultGateUpActivation,) if reference else _STRATEGIES,
            activation=activation, layout=layout, limit=limit,
        )

    def __call__(self, gate_up: torch.Tensor, up: torch.Tensor | None = None) -> torch.Tensor:
        return self.strategy(gate_up, up)

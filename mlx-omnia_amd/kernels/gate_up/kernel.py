"""The gate/up activation's contract.

The activation epilogue the reference's gate/up bindings share (core/layers.py:249-291,
core/kernels/gate_up/default.py:71-81): given the gate and up halves of a projection,
`act(gate) * up`. The declaration names the activation ("swiglu", or "swiglu_oai" with
its clamp `limit`, default.py:74-79) and how gate and up sit in the projection:
"blocked" (two tensors, or the halves [..., :I] and [..., I:] of one fused row) or
"interleaved" (pairs g0, u0, g1, u1, ... — SwitchGLU's load-time layout,
core/layers.py:275-287).
"""

from __future__ import annotations

from typing import Literal, Protocol, runtime_checkable

import torch

Activation = Literal["swiglu", "swiglu_oai"]
Layout = Literal["blocked", "interleaved"]


@runtime_checkable
class GateUpActivationStrategy(Protocol):
    def __call__(self, gate_up: torch.Tensor, up: torch.Tensor | None = None) -> torch.Tensor: ...


def split(gate_up: torch.Tensor, up: torch.Tensor | None, layout: Layout):
    """(gate, up) views of the declaration's operands."""
    if up is not None:
        return gate_up, up
    inner = gate_up.shape[-1] // 2
    if layout == "blocked":
        return gate_up[..., :inner], gate_up[..., inner:]
    pairs = gate_up.reshape(*gate_up.shape[:-1], inner, 2)
    return pairs[..., 0], pairs[..., 1]

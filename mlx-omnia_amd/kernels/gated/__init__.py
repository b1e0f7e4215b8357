"""Both gated activations of a layer, declared together: SwiGLU and the DeltaNet gate.

configs[3] pairs the SwiGLU `act(gate) * up` (core/layers.py:249-250,284-287; the
`GateUpActivation` facade here) with the gate `g = -exp(A_log) * softplus(a + dt_bias)`
(models/qwen3_5/layers/deltanet.py:222-224; the `GateSoftplus` facade). The gate is
1.5 MB at that config, so a launch of its own costs more than its bytes. A block that
declares both gets one dispatch for the pair:

- `HipGatedActivations` (`omnia_gated_activations`) binds where both `HipSwiGLU` and
  `HipGateSoftplus` bind, and computes exactly their arithmetic;
- `DefaultGatedActivations` runs the two Core chains.

`__call__(gate_up, up, a) -> (y, g)` takes the SwiGLU operands as `GateUpActivation`
does (two tensors, or one fused `[..., 2I]` row with `up=None`) and `a` as
`GateSoftplus` does. A call whose operands the fused kernel does not take (odd head
count, an odd row stride of `a`, operands the single kernels would hand to Core) runs the
two single bindings instead. That hand-off is recorded (`resolve.record_fallback`).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Protocol, runtime_checkable

import torch

from ...runtime import ops
from .._device import hip_device
from ..gate_softplus import DefaultGateSoftplus, HipGateSoftplus
from ..gate_up import DefaultGateUpActivation, HipSwiGLU, split
from ..gate_up.hip import applies as swiglu_applies
from ..resolve import record_fallback, resolve

__all__ = ["DefaultGatedActivations", "GatedActivations", "GatedActivationsStrategy",
           "HipGatedActivations"]


@runtime_checkable
class GatedActivationsStrategy(Protocol):
    def __call__(self, gate_up: torch.Tensor, up: torch.Tensor | None, a: torch.Tensor): ...


@dataclass(frozen=True)
class DefaultGatedActivations(GatedActivationsStrategy):
    activation: DefaultGateUpActivation
    gate: DefaultGateSoftplus

    @classmethod
    def build(cls, a_log, dt_bias, *, activation, layout, limit) -> "DefaultGatedActivations":
        return cls(DefaultGateUpActivation(activation, layout, limit),
                   DefaultGateSoftplus(a_log, dt_bias))

    def __call__(self, gate_up, up, a):
        return self.activation(gate_up, up), self.gate(a)


@dataclass(frozen=True)
class HipGatedActivations(GatedActivationsStrategy):
    swiglu: HipSwiGLU
    softplus: HipGateSoftplus

    @classmethod
    def build(cls, a_log, dt_bias, *, activation, layout, limit) -> "HipGatedActivations | None":
        swiglu = HipSwiGLU.build(activation=activation, layout=layout, limit=limit)
        softplus = HipGateSoftplus.build(a_log, dt_bias)
        if swiglu is None or softplus is None:
            return None
        return cls(swiglu, softplus)

    def __call__(self, gate_up, up, a):
        gate, up = split(gate_up, up, "blocked")
        heads = self.softplus.a_log.numel()
        served = (
            gate.dtype == torch.bfloat16 and up.dtype == torch.bfloat16
            and gate.shape == up.shape and swiglu_applies(gate.shape[-1])
            and a.dtype == torch.bfloat16 and a.shape[-1] == heads
            and hip_device(gate, up, a) and ops.gated_activations_applies(gate, up, a)
        )
        if not served:
            record_fallback(self, self.swiglu)
            return self.swiglu(gate, up), self.softplus(a)
        return ops.gated_activations(gate, up, a, self.softplus.a_log, self.softplus.dt_bias)


_STRATEGIES = (HipGatedActivations, DefaultGatedActivations)


class GatedActivations(GatedActivationsStrategy):
    """The layer's pair of gated activations: picks its binding once, then forwards."""

    def __init__(self, a_log: torch.Tensor, dt_bias: torch.Tensor, *, activation="swiglu",
                 layout="blocked", limit: float | None = None, reference: bool = False) -> None:
        self.strategy: GatedActivationsStrategy = resolve(
            (DefaultGatedActivations,) if reference else _STRATEGIES, a_log, dt_bias,
            activation=activation, layout=layout, limit=limit,
        )

    def __call__(self, gate_up: torch.Tensor, up: torch.Tensor | None, a: torch.Tensor):
        return self.strategy(gate_up, up, a)

"""The DeltaNet gate: `g = -exp(A_log) * softplus(a + dt_bias)`, one facade, two bindings.

In the reference this is two lines of model code (models/qwen3_5/layers/deltanet.py:
222-224; models/qwen3_next/layers/deltanet.py:122-123), consumed as exp(g) by the gated
delta step. Declared here as a primitive so a HIP binding can serve it: the declaration
is the per-head A_log and dt_bias (fp32 [heads]); the call takes a [..., heads] (bf16)
and returns g in fp32. `HipGateSoftplus` serves bf16 inputs on a gfx950 device;
`DefaultGateSoftplus` is the Core chain in torch ops.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Protocol, runtime_checkable

import torch

from ...runtime import ops
from .._device import hip_device
from ..resolve import record_fallback, resolve

__all__ = ["DefaultGateSoftplus", "GateSoftplus", "GateSoftplusStrategy", "HipGateSoftplus"]


@runtime_checkable
class GateSoftplusStrategy(Protocol):
    def __call__(self, a: torch.Tensor) -> torch.Tensor: ...


def softplus_core(dt: torch.Tensor) -> torch.Tensor:
    """mx.logaddexp(dt, 0): max + log1p(exp(min - max)), with its infinite arms."""
    maxval = torch.clamp(dt, min=0.0)
    minval = torch.clamp(dt, max=0.0)
    value = maxval + torch.log1p(torch.exp(minval - maxval))
    return torch.where((minval == -torch.inf) | (maxval == torch.inf), maxval, value)


@dataclass(frozen=True)
class DefaultGateSoftplus(GateSoftplusStrategy):
    a_log: torch.Tensor
    dt_bias: torch.Tensor

    @classmethod
    def build(cls, a_log, dt_bias) -> "DefaultGateSoftplus":
        return cls(a_log, dt_bias)

    def __call__(self, a: torch.Tensor) -> torch.Tensor:
        dt = a.float() + self.dt_bias.float()
        return -torch.exp(self.a_log.float()) * softplus_core(dt)


@dataclass(frozen=True)
class HipGateSoftplus(GateSoftplusStrategy):
    a_log: torch.Tensor
    dt_bias: torch.Tensor
    fallback: DefaultGateSoftplus

    @classmethod
    def build(cls, a_log, dt_bias) -> "HipGateSoftplus | None":
        if a_log.dim() != 1 or a_log.shape != dt_bias.shape:
            return None
        if not hip_device(a_log, dt_bias):
            return None
        return cls(a_log.float().contiguous(), dt_bias.float().contiguous(),
                   DefaultGateSoftplus(a_log, dt_bias))

    def __call__(self, a: torch.Tensor) -> torch.Tensor:
        if a.dtype != torch.bfloat16 or a.shape[-1] != self.a_log.numel() or a.stride(-1) != 1:
            record_fallback(self, self.fallback)
            return self.fallback(a)
        return ops.gate_softplus(a, self.a_log, self.dt_bias)


_STRATEGIES = (HipGateSoftplus, DefaultGateSoftplus)


class GateSoftplus(GateSoftplusStrategy):
    def __init__(self, a_log: torch.Tensor, dt_bias: torch.Tensor, *, reference: bool = False) -> None:
        self.strategy: GateSoftplusStrategy = resolve(
            (DefaultGateSoftplus,) if reference else _STRATEGIES, a_log, dt_bias
        )

    def __call__(self, a: torch.Tensor) -> torch.Tensor:
        return self.strategy(a)

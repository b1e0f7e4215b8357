"""SwiGLU in one HIP dispatch (`omnia_swiglu`, csrc/activations.hip).

Serves the plain "swiglu" activation over blocked gate/up (two tensors or the halves of
a fused row) in bf16; a clamp (`limit`), the swiglu_oai variant and the interleaved
layout are other arithmetic or another layout and decline to the Core chain. Operands
the kernel does not take (not on a gfx950 device, another dtype, rows that are not
16-byte vectors) go to the Core fallback, as the reference's kernels fall back on the
shapes they do not serve.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ...runtime import ops
from ..resolve import record_fallback
from .._device import hip_device
from .default import DefaultGateUpActivation
from .kernel import GateUpActivationStrategy, split


def applies(inner: int) -> bool:
    return inner > 0 and inner % 8 == 0


@dataclass(frozen=True)
class HipSwiGLU(GateUpActivationStrategy):
    fallback: DefaultGateUpActivation

    @classmethod
    def build(cls, *, activation, layout, limit) -> "HipSwiGLU | None":
        if activation != "swiglu" or limit is not None or layout != "blocked":
            return None
        return cls(DefaultGateUpActivation(activation, layout, limit))

    def __call__(self, gate_up: torch.Tensor, up: torch.Tensor | None = None) -> torch.Tensor:
        gate, up = split(gate_up, up, "blocked")
        served = (
            gate.dtype == torch.bfloat16 and up.dtype == torch.bfloat16
            and gate.shape == up.shape and applies(gate.shape[-1])
        )
        if not served or not hip_device(gate, up):
            record_fallback(self, self.fallback)
            return self.fallback(gate, up)
        return ops.swiglu(gate, up)

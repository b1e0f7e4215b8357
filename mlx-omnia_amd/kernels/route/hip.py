"""The HIP routing strategies (csrc/router.hip), over logits from the stock matmul or
the caller:

- `HipSoftmaxTopkRoute` (`omnia_softmax_topk_slots`): softmax -> top-k, the
  declarations core/kernels/route/softmax_topk.py:295-336 (`SoftmaxTopkRoute.build`)
  serves for the softmax family (no bias, no scale, no softcap), renormalised with no
  epsilon, with or without the shared expert's sigmoid slot (softmax_topk.py:67-72,
  Qwen3.5's declaration), and also `normalize=False` (the Core chain's arm,
  core/kernels/route/default.py:62-63, Qwen3's `normalize=norm_topk`), with the
  lowest-index tie rule, up to 256 experts and k <= 64 (63 with the shared slot);
- `HipOrdinalRoute` (`omnia_sigmoid_topk`): sigmoid scoring with a correction bias,
  ordinal keys, lower-index ties and weights from the unbiased scores, where
  core/kernels/route/ordinal.py:265-286 (`OrdinalRoute.build`) binds: renormalise with
  no epsilon, no scale, no shared slot, no hash table, no softcap, and the tournament's
  shape (`router_tournament_applies`, ordinal.py:158-174).

A call whose logits the kernel does not take (not bf16 or fp32, or not on the device)
goes to the Core chain and is recorded (`resolve.record_fallback`).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ...runtime import ops
from .._device import hip_device
from ..resolve import record_fallback
from .default import DefaultRoute
from .kernel import RouteStrategy, Routing, gate_logits


def softmax_topk_applies(experts: int, k: int, shared: bool = False) -> bool:
    return 0 < experts <= 256 and 0 < k <= min(experts, 63 if shared else 64)


@dataclass(frozen=True)
class HipSoftmaxTopkRoute(RouteStrategy):
    gate: torch.Tensor | None
    routing: Routing
    fallback: DefaultRoute

    @classmethod
    def build(cls, gate, *, routing: Routing) -> "HipSoftmaxTopkRoute | None":
        if not routing.softmax_slots() or not softmax_topk_applies(routing.experts, routing.k,
                                                                    routing.shared):
            return None
        if gate is not None and not hip_device(gate):
            return None
        return cls(gate, routing, DefaultRoute(gate, routing))

    def __call__(self, row, *, logits=None, ids=None):
        routing = self.routing
        values = gate_logits(self.gate, row, logits)
        width = routing.experts + (1 if routing.shared else 0)
        if values.dtype != torch.bfloat16 or values.shape[-1] != width or not hip_device(values):
            record_fallback(self, self.fallback)
            return self.fallback(row, logits=values)
        return ops.softmax_topk(values, routing.k, normalize=routing.normalize,
                                shared=routing.shared)

    def rows(self, logits: torch.Tensor):
        return self(logits, logits=logits)


def ordinal_route_applies(experts: int, k: int) -> bool:
    """ordinal.py:158-174: 32-expert blocks and a 64-candidate merge."""
    return (experts % 32 == 0 and 32 <= experts <= 1024 and 0 < k <= 32
            and (experts // 32) * k == 64)


def sigmoid_bias_routing(routing: Routing) -> bool:
    """Sigmoid scores with a correction bias, renormalised over the winners, nothing else
    (the declaration ordinal.py:265-277 builds for), lower-index ties."""
    return (
        routing.scoring == "sigmoid" and routing.bias is not None and routing.normalize
        and routing.norm_eps == 0.0 and routing.scale == 1.0 and not routing.shared
        and routing.hash_table is None and routing.softcap == 0.0 and routing.ties == "lower"
    )


@dataclass(frozen=True)
class HipOrdinalRoute(RouteStrategy):
    gate: torch.Tensor | None
    routing: Routing
    bias: torch.Tensor
    fallback: DefaultRoute

    @classmethod
    def build(cls, gate, *, routing: Routing) -> "HipOrdinalRoute | None":
        if not sigmoid_bias_routing(routing) or not ordinal_route_applies(routing.experts, routing.k):
            return None
        bias = routing.bias
        if bias.dtype != torch.float32 or bias.numel() != routing.experts or not hip_device(bias):
            return None
        if gate is not None and not hip_device(gate):
            return None
        return cls(gate, routing, bias.contiguous(), DefaultRoute(gate, routing))

    def __call__(self, row, *, logits=None, ids=None):
        values = gate_logits(self.gate, row, logits)
        if (values.dtype not in (torch.bfloat16, torch.float32)
                or values.shape[-1] != self.routing.experts or not hip_device(values)):
            record_fallback(self, self.fallback)
            return self.fallback(row, logits=values)
        indices, weights, _ = ops.sigmoid_topk(values.contiguous(), self.bias, self.routing.k)
        return indices, weights

    def rows(self, logits: torch.Tensor):
        return self(logits, logits=logits)

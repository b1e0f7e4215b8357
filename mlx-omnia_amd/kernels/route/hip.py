"""softmax -> top-k -> renormalise over many rows in one HIP dispatch
(`omnia_softmax_topk`, csrc/router.hip).

Serves the declarations core/kernels/route/softmax_topk.py:295-336
(`SoftmaxTopkRoute.build`) serves for the softmax family — no bias, renormalise with no
epsilon, no scale, no softcap — without a shared slot, with the lowest-index tie rule,
up to 256 experts and k <= 64. The logits come from the stock matmul (or the caller).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ...runtime import ops
from .._device import hip_device
from .default import DefaultRoute
from .kernel import RouteStrategy, Routing, gate_logits


def softmax_topk_applies(experts: int, k: int) -> bool:
    return 0 < experts <= 256 and 0 < k <= min(experts, 64)


@dataclass(frozen=True)
class HipSoftmaxTopkRoute(RouteStrategy):
    gate: torch.Tensor | None
    routing: Routing
    fallback: DefaultRoute

    @classmethod
    def build(cls, gate, *, routing: Routing) -> "HipSoftmaxTopkRoute | None":
        if not routing.plain_softmax() or not softmax_topk_applies(routing.experts, routing.k):
            return None
        if gate is not None and not hip_device(gate):
            return None
        return cls(gate, routing, DefaultRoute(gate, routing))

    def __call__(self, row, *, logits=None, ids=None):
        values = gate_logits(self.gate, row, logits)
        if (values.dtype != torch.bfloat16 or values.shape[-1] != self.routing.experts
                or not hip_device(values)):
            return self.fallback(row, logits=values)
        return ops.softmax_topk(values, self.routing.k)

    def rows(self, logits: torch.Tensor):
        return self(logits, logits=logits)

"""The residual join fused with the router: add + RMSNorm + router projection + top-k.

core/kernels/route/residual.py:117-299 fuses the one-token residual join with the router
gemv (sigmoid scoring, ordinal keys) as machinery beside the routing strategies. Here the
same fusion is a facade of its own, declared by the norm leaf (`.weight`, `.eps`), the
router gate [experts, hidden] and a `Routing`, and called as
`(x, projected) -> (summed, normalized, indices, weights)`. `HipResidualRouter` serves
softmax routing at hidden 2048 or 4096 and 128 or 256 experts in one dispatch
(`omnia_residual_rms_router`, csrc/router.hip); it repacks the gate once when it is
built (`omnia_pack_router_weight`), as the reference's strategies take their weights at
build. `DefaultResidualRouter` is the Core chain (the residual join, the gate matmul,
the routing chain).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Protocol, runtime_checkable

import torch

from ...runtime import ops
from .._device import hip_device
from ..add_norm import AddRmsNorm
from ..resolve import resolve
from .default import DefaultRoute
from .kernel import Routing


@runtime_checkable
class ResidualRouterStrategy(Protocol):
    def __call__(self, x: torch.Tensor, projected: torch.Tensor): ...


def residual_router_applies(hidden: int, experts: int, k: int) -> bool:
    return hidden in (2048, 4096) and experts in (128, 256) and 0 < k <= 64


@dataclass(frozen=True)
class DefaultResidualRouter(ResidualRouterStrategy):
    join: AddRmsNorm
    route: DefaultRoute

    @classmethod
    def build(cls, leaf, gate, *, routing: Routing) -> "DefaultResidualRouter":
        return cls(AddRmsNorm(leaf, reference=True), DefaultRoute(gate, routing))

    def __call__(self, x, projected):
        summed, normalized = self.join(x, projected)
        logits = normalized @ self.route.gate.T
        indices, weights = self.route(normalized, logits=logits)
        return summed, normalized, indices, weights


@dataclass(frozen=True)
class HipResidualRouter(ResidualRouterStrategy):
    norm_weight: torch.Tensor
    eps: float
    gate: ops.PackedRouterWeight
    routing: Routing

    @classmethod
    def build(cls, leaf, gate, *, routing: Routing) -> "HipResidualRouter | None":
        weight = leaf.weight
        if not routing.plain_softmax() or gate.shape[0] != routing.experts:
            return None
        if not residual_router_applies(weight.numel(), routing.experts, routing.k):
            return None
        if weight.dtype != torch.bfloat16 or gate.dtype != torch.bfloat16:
            return None
        if not hip_device(weight, gate):
            return None
        return cls(weight.contiguous(), float(leaf.eps), ops.pack_router_weight(gate.contiguous()),
                   routing)

    def __call__(self, x, projected):
        summed, normalized, _, indices, weights = ops.residual_rms_router(
            x.contiguous(), projected.contiguous(), self.norm_weight, self.gate,
            k=self.routing.k, eps=self.eps,
        )
        return summed, normalized, indices, weights


_STRATEGIES = (HipResidualRouter, DefaultResidualRouter)


class ResidualRouter(ResidualRouterStrategy):
    def __init__(self, leaf, gate: torch.Tensor, *, routing: Routing, reference: bool = False) -> None:
        self.strategy: ResidualRouterStrategy = resolve(
            (DefaultResidualRouter,) if reference else _STRATEGIES, leaf, gate, routing=routing
        )

    def __call__(self, x, projected):
        return self.strategy(x, projected)

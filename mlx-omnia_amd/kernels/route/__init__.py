"""MoE routing: the `Route` facade over router logits and the fused `ResidualRouter`.

Mirrors core/kernels/route/__init__.py:48-100: a block declares its routing and `Route`
binds the first strategy whose `build` accepts it. `HipSoftmaxTopkRoute` serves plain
softmax routing (lowest-index ties) on a gfx950 device, `HipOrdinalRoute` sigmoid
routing with a correction bias where the reference's `OrdinalRoute` binds;
`DefaultRoute` (the Core chain) serves every declaration.
"""

from __future__ import annotations

import torch

from ..resolve import resolve
from .default import DefaultRoute, ordinal_keys, top_k
from .hip import (HipOrdinalRoute, HipSoftmaxTopkRoute, ordinal_route_applies,
                  sigmoid_bias_routing, softmax_topk_applies)
from .kernel import RouteStrategy, Routing, Scoring, Ties, gate_logits
from .residual import (
    DefaultResidualRouter,
    HipResidualRouter,
    ResidualRouter,
    residual_router_applies,
)

__all__ = [
    "DefaultResidualRouter",
    "DefaultRoute",
    "HipOrdinalRoute",
    "HipResidualRouter",
    "HipSoftmaxTopkRoute",
    "ResidualRouter",
    "Route",
    "RouteStrategy",
    "Routing",
    "Scoring",
    "Ties",
    "gate_logits",
    "ordinal_keys",
    "ordinal_route_applies",
    "residual_router_applies",
    "sigmoid_bias_routing",
    "softmax_topk_applies",
    "top_k",
]

_STRATEGIES = (HipSoftmaxTopkRoute, HipOrdinalRoute, DefaultRoute)


class Route(RouteStrategy):
    """The routing a block declares: picks its binding once, then forwards every call."""

    def __init__(
        self,
        gate: torch.Tensor | None,
        *,
        experts: int,
        k: int,
        scoring: Scoring = "softmax",
        bias: torch.Tensor | None = None,
        normalize: bool = True,
        norm_eps: float = 0.0,
        scale: float = 1.0,
        softcap: float = 0.0,
        shared: bool = False,
        hash_table: torch.Tensor | None = None,
        ties: Ties = "lower",
        reference: bool = False,
    ) -> None:
        self.routing = Routing(experts=experts, k=k, scoring=scoring, bias=bias,
                               normalize=normalize, norm_eps=norm_eps, scale=scale,
                               softcap=softcap, shared=shared, hash_table=hash_table, ties=ties)
        self.strategy: RouteStrategy = resolve(
            (DefaultRoute,) if reference else _STRATEGIES, gate, routing=self.routing
        )

    def __call__(self, row, *, logits=None, ids=None):
        return self.strategy(row, logits=logits, ids=ids)

    def rows(self, logits: torch.Tensor):
        return self.strategy.rows(logits)

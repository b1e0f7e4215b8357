"""The residual join fused with the router: add + RMSNorm + router projection + top-k.

core/kernels/route/residual.py:117-299 fuses the one-token residual join with the router
gemv (sigmoid scoring, ordinal keys) as machinery beside the routing strategies. Here the
same fusion is a facade of its own, declared by the norm leaf (`.weight`, `.eps`), the
router gate [experts, hidden] and a `Routing`, and called as
`(x, projected) -> (summed, normalized, indices, weights)`, or as `with_keys(x, projected)
-> (summed, normalized, logits, keys)`, the reference's own return (residual.py:268-299)
for a sigmoid declaration with a correction bias. `HipResidualRouter` serves softmax
routing (`omnia_residual_rms_router`) and sigmoid routing with a correction bias
(`omnia_residual_rms_router_sigmoid`) at hidden 2048 or 4096 and 128 or 256 experts in
one dispatch (csrc/router.hip); it repacks the gate once when it is built
(`omnia_pack_router_weight`), as the reference's strategies take their weights at build.
`DefaultResidualRouter` is the Core chain (the residual join, the gate matmul, the
routing chain, and the ordinal keys of ordinal.py:253-262 in torch ops).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Protocol, runtime_checkable

import torch

from ...runtime import ops
from .._device import hip_device
from ..add_norm import AddRmsNorm
from ..resolve import resolve
from .default import DefaultRoute, ordinal_keys
from .hip import sigmoid_bias_routing
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

    def with_keys(self, x, projected):
        routing = self.route.routing
        assert routing.scoring == "sigmoid" and routing.bias is not None
        summed, normalized = self.join(x, projected)
        logits = normalized @ self.route.gate.T
        keys = ordinal_keys(torch.sigmoid(logits.float()) + routing.bias)
        return summed, normalized, logits, keys


@dataclass(frozen=True)
class HipResidualRouter(ResidualRouterStrategy):
    norm_weight: torch.Tensor
    eps: float
    gate: ops.PackedRouterWeight
    routing: Routing

    @classmethod
    def build(cls, leaf, gate, *, routing: Routing) -> "HipResidualRouter | None":
        weight = leaf.weight
        sigmoid = sigmoid_bias_routing(routing)
        if not (routing.plain_softmax() or sigmoid) or gate.shape[0] != routing.experts:
            return None
        if sigmoid and (routing.bias.dtype != torch.float32 or routing.bias.numel() != routing.experts
                        or not hip_device(routing.bias)):
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
        # Up to 64 tokens (decode steps, short prefills) take the library's decode path,
        # which needs the logits written out; more tokens run the one fused dispatch
        # without them.
        decode = x.numel() // x.shape[-1] <= ops.ROUTER_SELECT_VIA_DECODE_ROWS
        if self.routing.bias is not None:
            summed, normalized, _, _, indices, weights = ops.residual_rms_router_sigmoid(
                x.contiguous(), projected.contiguous(), self.norm_weight, self.gate,
                self.routing.bias.contiguous(), k=self.routing.k, eps=self.eps,
                emit_logits=decode, emit_keys=False, select=True,
            )
            return summed, normalized, indices, weights
        summed, normalized, _, indices, weights = ops.residual_rms_router(
            x.contiguous(), projected.contiguous(), self.norm_weight, self.gate,
            k=self.routing.k, eps=self.eps, emit_logits=decode,
        )
        return summed, normalized, indices, weights

    def with_keys(self, x, projected):
        assert self.routing.bias is not None, "with_keys: a sigmoid declaration with a bias"
        summed, normalized, logits, keys, _, _ = ops.residual_rms_router_sigmoid(
            x.contiguous(), projected.contiguous(), self.norm_weight, self.gate,
            self.routing.bias.contiguous(), k=self.routing.k, eps=self.eps,
        )
        return summed, normalized, logits, keys


_STRATEGIES = (HipResidualRouter, DefaultResidualRouter)


class ResidualRouter(ResidualRouterStrategy):
    def __init__(self, leaf, gate: torch.Tensor, *, routing: Routing, reference: bool = False) -> None:
        self.strategy: ResidualRouterStrategy = resolve(
            (DefaultResidualRouter,) if reference else _STRATEGIES, leaf, gate, routing=routing
        )

    def __call__(self, x, projected):
        return self.strategy(x, projected)

    def with_keys(self, x, projected):
        """(summed, normalized, logits, keys) of a sigmoid declaration with a bias."""
        return self.strategy.with_keys(x, projected)

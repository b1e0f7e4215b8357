"""The Core routing strategy: the declaration spelled out in torch ops
(core/kernels/route/default.py:24-69). Accepts every declaration, so it registers last."""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .kernel import RouteStrategy, Routing, gate_logits


def top_k(scores: torch.Tensor, k: int, ties: str) -> torch.Tensor:
    """Indices of the k largest scores, descending; exact ties by the declared rule."""
    if ties == "lower":
        return torch.sort(scores, dim=-1, descending=True, stable=True).indices[..., :k]
    # Higher index first among equals: a stable sort of the reversed row.
    experts = scores.shape[-1]
    flipped = torch.sort(scores.flip(-1), dim=-1, descending=True, stable=True).indices[..., :k]
    return experts - 1 - flipped


def ordinal_keys(biased: torch.Tensor) -> torch.Tensor:
    """core/kernels/route/ordinal.py:253-262 in torch ops: the keys whose ascending
    unsigned order is the descending order of the biased scores (uint32)."""
    bits = (-biased.float()).view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    negative = (bits & 0x80000000) != 0
    return torch.where(negative, (~bits) & 0xFFFFFFFF, bits ^ 0x80000000).to(torch.uint32)


@dataclass(frozen=True)
class DefaultRoute(RouteStrategy):
    gate: torch.Tensor | None
    routing: Routing

    @classmethod
    def build(cls, gate, *, routing: Routing) -> "DefaultRoute":
        return cls(gate, routing)

    def __call__(self, row, *, logits=None, ids=None):
        routing = self.routing
        values = gate_logits(self.gate, row, logits)
        if routing.softcap > 0.0:
            values = torch.tanh(values / routing.softcap) * routing.softcap
        routed = values[..., : routing.experts]
        if routing.scoring == "softmax":
            scores = torch.softmax(routed.float(), dim=-1)
        elif routing.scoring == "sigmoid":
            scores = torch.sigmoid(routed.float())
        else:
            scores = torch.sqrt(F.softplus(routed.float()))
        if routing.hash_table is not None:
            assert ids is not None
            chosen = routing.hash_table[ids].reshape(*scores.shape[:-1], -1).long()
        else:
            biased = scores if routing.bias is None else scores + routing.bias
            # Sort on the logits for softmax (monotone): exact ties are exact.
            key = routed.float() if routing.scoring == "softmax" and routing.bias is None else biased
            chosen = top_k(key, routing.k, routing.ties)
        weights = torch.gather(scores, -1, chosen)
        if routing.normalize:
            weights = weights / (weights.sum(dim=-1, keepdim=True) + routing.norm_eps)
        weights = weights * routing.scale
        chosen = chosen.to(torch.int32)
        if routing.shared:
            slot = torch.full((*chosen.shape[:-1], 1), routing.experts, dtype=torch.int32,
                              device=chosen.device)
            shared = torch.sigmoid(values[..., routing.experts :].float())
            return torch.cat([chosen, slot], -1), torch.cat([weights, shared], -1)
        return chosen, weights

    def rows(self, logits: torch.Tensor):
        return self(logits, logits=logits)

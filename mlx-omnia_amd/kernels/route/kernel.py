"""The routing primitive's contract (core/kernels/route/kernel.py:22-82).

`Routing` is the declaration every strategy's `build` reads in full: a strategy builds
only when it computes exactly the declared chain. One knob is added to the reference's:
`ties`, the rule for exactly equal scores. "lower" (lowest expert index first, the rule
of core/kernels/route/ordinal.py:1-27) is what this build's kernels compute; "higher"
is the reference softmax chain's rule (core/kernels/route/default.py:7-9, mlx's stable
ascending argpartition), served by the Core strategy only.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal, Protocol, runtime_checkable

import torch

Scoring = Literal["softmax", "sigmoid", "sqrt_softplus"]
Ties = Literal["lower", "higher"]


@dataclass(frozen=True)
class Routing:
    experts: int
    k: int
    scoring: Scoring = "softmax"
    bias: torch.Tensor | None = None
    normalize: bool = True
    norm_eps: float = 0.0
    scale: float = 1.0
    softcap: float = 0.0
    shared: bool = False
    hash_table: torch.Tensor | None = None
    ties: Ties = "lower"

    @property
    def slots(self) -> int:
        return self.k + (1 if self.shared else 0)

    def plain_softmax(self) -> bool:
        """softmax -> top-k -> renormalise, nothing else (what the fused router computes)."""
        return self.softmax_slots() and self.normalize and not self.shared

    def softmax_slots(self) -> bool:
        """Softmax scoring with no bias, scale, softcap or hash table and the lower-index
        tie rule; renormalised with no epsilon or not at all; with or without the shared
        slot (what `omnia_softmax_topk_slots` computes)."""
        return (
            self.scoring == "softmax" and self.bias is None and self.norm_eps == 0.0
            and self.scale == 1.0 and self.softcap == 0.0 and self.hash_table is None
            and self.ties == "lower"
        )


@runtime_checkable
class RouteStrategy(Protocol):
    """(row [..., hidden]) -> (indices [..., slots] int32, weights [..., slots])."""

    def __call__(self, row: torch.Tensor, *, logits: torch.Tensor | None = None,
                 ids: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]: ...


def gate_logits(gate: torch.Tensor | None, row: torch.Tensor,
                logits: torch.Tensor | None) -> torch.Tensor:
    """Router logits [..., E] from the gate [E, hidden] or the caller's own
    (core/kernels/route/kernel.py:75-82)."""
    if logits is not None:
        return logits
    assert gate is not None
    return row @ gate.T

"""The residual join — add plus the RMSNorm that reads it — one facade, two bindings.

Mirrors core/kernels/add_norm/__init__.py:36-53: a block declares the norm leaf (any
object with `.weight` and `.eps`) and how many tokens it hands over; `AddRmsNorm`
binds the first strategy whose `build` accepts the declaration. `HipAddRmsNorm` serves
bf16 rows on a gfx950 device; `DefaultAddRmsNorm` (the Core chain) serves everything
else and is what `reference=True` forces.
"""

from __future__ import annotations

import torch

from ..resolve import resolve
from .default import DefaultAddRmsNorm, rms_norm_core
from .hip import HipAddRmsNorm, applies
from .kernel import AddRmsNormStrategy

__all__ = [
    "AddRmsNorm",
    "AddRmsNormStrategy",
    "DefaultAddRmsNorm",
    "HipAddRmsNorm",
    "applies",
    "rms_norm_core",
]

# The HIP kernel first; the Core chain after it takes any declaration.
_STRATEGIES = (HipAddRmsNorm, DefaultAddRmsNorm)


class AddRmsNorm(AddRmsNormStrategy):
    """The join a block declares: picks its binding once, then forwards every call."""

    def __init__(self, leaf, *, tokens: int | None = None, reference: bool = False) -> None:
        self.strategy: AddRmsNormStrategy = resolve(
            (DefaultAddRmsNorm,) if reference else _STRATEGIES, leaf, tokens=tokens
        )

    def __call__(
        self, x: torch.Tensor, projected: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]:
        return self.strategy(x, projected)

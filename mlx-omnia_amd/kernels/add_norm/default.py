"""The Core residual-join strategy: the add and the norm as two torch ops.

Restates core/kernels/add_norm/default.py:18-29 (`x + p`, then `mx.fast.rms_norm`) with
mx.fast.rms_norm's rounding points (core/kernels/add_norm/rows.py:3-9,75-79): the sum is
rounded to the input dtype once, the normalised value is rounded to the dtype *before*
the weight multiplies it, and the product is rounded again. `build` accepts every
declaration, so it registers last and makes the facade total.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .kernel import AddRmsNormStrategy


def rms_norm_core(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """`w * T(x * rsqrt(mean(x^2) + eps))` over the last axis, fp32 inside."""
    wide = x.float()
    inv = 1.0 / torch.sqrt((wide * wide).mean(dim=-1, keepdim=True) + eps)
    return (weight.float() * (wide * inv).to(x.dtype).float()).to(x.dtype)


@dataclass(frozen=True)
class DefaultAddRmsNorm(AddRmsNormStrategy):
    weight: torch.Tensor
    eps: float

    @classmethod
    def build(cls, leaf, *, tokens: int | None) -> "DefaultAddRmsNorm":
        return cls(leaf.weight, float(leaf.eps))

    def __call__(
        self, x: torch.Tensor, projected: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]:
        added = x + projected
        return added, rms_norm_core(added, self.weight, self.eps)

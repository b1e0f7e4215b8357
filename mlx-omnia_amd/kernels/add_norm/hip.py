"""Residual add + RMSNorm over any number of rows in one HIP dispatch.

Serves the declarations core/kernels/add_norm/rows.py:106-128 (`RowsAddRmsNorm`, any T)
and core/kernels/add_norm/fused.py:99-120 (`FusedAddRmsNorm`, T=1) serve in the
reference, with the Core chain's rounding for every T: the fused.py single-token path
keeps `s * inv * w` in fp32, a different numerical path that is not the declared Core
arithmetic and is not reproduced. Kernel: `omnia_add_rms_norm`
(csrc/add_rms_norm.hip), one wave64 per row.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ...runtime import ops
from .._device import hip_device
from .kernel import AddRmsNormStrategy

MAX_HIDDEN = 8192


def applies(hidden: int) -> bool:
    """The row tiles as 16-byte vectors, at most 16 per lane of one wave64."""
    return hidden > 0 and hidden % 8 == 0 and hidden <= MAX_HIDDEN


@dataclass(frozen=True)
class HipAddRmsNorm(AddRmsNormStrategy):
    weight: torch.Tensor
    eps: float

    @classmethod
    def build(cls, leaf, *, tokens: int | None) -> "HipAddRmsNorm | None":
        weight = leaf.weight
        if weight.dtype != torch.bfloat16 or not applies(weight.numel()):
            return None
        if not hip_device(weight):
            return None
        return cls(weight.contiguous(), float(leaf.eps))

    def __call__(
        self, x: torch.Tensor, projected: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]:
        return ops.add_rms_norm(x.contiguous(), projected.contiguous(), self.weight, self.eps)

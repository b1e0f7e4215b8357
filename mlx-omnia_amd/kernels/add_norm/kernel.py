"""The residual-join primitive's contract (core/kernels/add_norm/kernel.py:15-19).

(x [..., hidden], projected [..., hidden]) -> (x + projected, rms_norm of that sum), both
keeping the input's shape and dtype.
"""

from __future__ import annotations

from typing import Protocol, runtime_checkable

import torch


@runtime_checkable
class AddRmsNormStrategy(Protocol):
    def __call__(
        self, x: torch.Tensor, projected: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor]: ...

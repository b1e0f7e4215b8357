"""The device gate every HIP strategy's `build` passes through."""

from __future__ import annotations

import torch

from ..runtime import library
from ..runtime.ops import on_rocm


def hip_device(*tensors: torch.Tensor) -> bool:
    """True when every tensor sits on one ROCm device and the HIP library is loaded.

    Tensors elsewhere (CPU) decline, so the Core strategy serves them. A ROCm-resident
    declaration with the library missing raises `LibraryMissing` instead of declining:
    a GPU declaration never lands on the Core chain because a build step was skipped.
    """
    if not on_rocm(*tensors):
        return False
    library()
    return True

"""Torch-facing calls into the C ABI.

Each function checks what the kernel assumes (device, dtype, contiguity, shape),
allocates the outputs with torch on the inputs' device unless the caller passes them,
and enqueues the kernel on the current torch stream of that device. The checks run on
the host before anything is launched, so a kernel never sees a shape its grid does not
fit.
"""

from __future__ import annotations

import torch

from .loader import call

BF16 = torch.bfloat16
F32 = torch.float32


def on_rocm(*tensors: torch.Tensor) -> bool:
    """All tensors live on one ROCm device."""
    if torch.version.hip is None or not tensors:
        return False
    device = tensors[0].device
    return all(t.is_cuda and t.device == device for t in tensors)


def _require(condition: bool, message: str) -> None:
    if not condition:
        raise ValueError(message)


def _dense(t: torch.Tensor, dtype: torch.dtype, name: str) -> None:
    _require(t.dtype == dtype, f"{name}: expected {dtype}, got {t.dtype}")
    _require(t.is_contiguous(), f"{name}: must be contiguous")
    _require(t.data_ptr() % 16 == 0 or t.numel() == 0, f"{name}: must be 16-byte aligned")


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _out(out: torch.Tensor | None, like: torch.Tensor, shape, dtype, name: str) -> torch.Tensor:
    if out is None:
        return torch.empty(shape, dtype=dtype, device=like.device)
    _require(tuple(out.shape) == tuple(shape), f"{name}: shape {tuple(out.shape)} != {tuple(shape)}")
    _dense(out, dtype, name)
    _require(out.device == like.device, f"{name}: wrong device")
    return out


def add_rms_norm(
    x: torch.Tensor,
    branch: torch.Tensor,
    weight: torch.Tensor,
    eps: float,
    *,
    summed: torch.Tensor | None = None,
    normalized: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """`(x + branch, rms_norm(x + branch))` over the last axis; see `omnia_add_rms_norm`."""
    hidden = weight.numel()
    _require(on_rocm(x, branch, weight), "add_rms_norm: tensors must share one ROCm device")
    _require(x.shape == branch.shape and x.shape[-1] == hidden, "add_rms_norm: shape mismatch")
    for t, name in ((x, "x"), (branch, "branch"), (weight, "weight")):
        _dense(t, BF16, name)
    summed = _out(summed, x, x.shape, BF16, "summed")
    normalized = _out(normalized, x, x.shape, BF16, "normalized")
    rows = x.numel() // hidden if hidden else 0
    call(
        "omnia_add_rms_norm",
        x.data_ptr(), branch.data_ptr(), weight.data_ptr(),
        summed.data_ptr(), normalized.data_ptr(),
        rows, hidden, float(eps), _stream(x),
    )
    return summed, normalized

"""The T=1 unrouted SwiGLU MLP: (row [hidden], residual [hidden]) -> [hidden].

Mirrors core/kernels/mlp/__init__.py and kernel.py (`Mlp`, `MlpStrategy`, `Activation`):
a block declares the leaf (a `SwiGLU` with `gate_up_proj` [2I, H] and `down_proj`
[H, I], gate rows first) and its activation, and the first strategy whose `build`
accepts the declaration serves it.

- `HipDenseMlp` serves what the reference's `DenseMlp` serves (core/kernels/mlp/dense.py:
  222-246): bf16 `nn.Linear` projections without bias, silu, in two dispatches
  (`omnia_dense_gate_up_swiglu`, then `omnia_dense_down_residual`, csrc/mlp.hip), with the
  reference's bf16 SwiGLU chain (every temporary rounded to bf16) and the residual add
  rounded once.
- `DefaultMlp` is the Core chain (core/kernels/mlp/default.py:20-29): the leaf called as
  the layer it is, then the residual add in torch ops. It accepts everything.

The reference also registers an nvfp4 strategy ahead of the dense one; quantised leaves
are not built here, so they land on `DefaultMlp`.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal, Protocol, runtime_checkable

import torch

from ...runtime import ops
from .._device import hip_device
from ..resolve import resolve

Activation = Literal["silu", "gelu_tanh"]

__all__ = ["Activation", "DefaultMlp", "HipDenseMlp", "Mlp", "MlpStrategy",
           "dense_down_residual_applies", "dense_gate_up_swiglu_applies"]


@runtime_checkable
class MlpStrategy(Protocol):
    def __call__(self, row: torch.Tensor, residual: torch.Tensor) -> torch.Tensor: ...


def dense_gate_up_swiglu_applies(hidden: int, inner: int) -> bool:
    """x stays packed in registers: hidden / 8 16-byte vectors, at most 16 per lane. (The
    reference's Metal tiling asks hidden % 128 == 0 and inner % 64 == 0; this kernel
    bounds-checks its rows and needs neither.)"""
    return 0 < hidden <= 8192 and hidden % 8 == 0 and inner > 0


def dense_down_residual_applies(hidden: int, inner: int) -> bool:
    """Rows of 16-byte vectors: inner % 8 == 0 (the reference's: inner % 128, hidden % 16)."""
    return hidden > 0 and inner > 0 and inner % 8 == 0


@dataclass(frozen=True)
class DefaultMlp(MlpStrategy):
    leaf: torch.nn.Module

    @classmethod
    def build(cls, leaf, *, hidden, inner, activation) -> "DefaultMlp":
        return cls(leaf)

    def __call__(self, row: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
        return self.leaf(row[None]).reshape(-1) + residual


@dataclass(frozen=True)
class HipDenseMlp(MlpStrategy):
    fused_weight: torch.Tensor
    down_weight: torch.Tensor

    @classmethod
    def build(cls, leaf, *, hidden, inner, activation) -> "HipDenseMlp | None":
        gate_up = getattr(leaf, "gate_up_proj", None)
        down = getattr(leaf, "down_proj", None)
        if activation != "silu":
            return None
        if not isinstance(gate_up, torch.nn.Linear) or not isinstance(down, torch.nn.Linear):
            return None
        if gate_up.bias is not None or down.bias is not None:
            return None
        fused, down_w = gate_up.weight, down.weight
        if fused.dtype != torch.bfloat16 or down_w.dtype != torch.bfloat16:
            return None
        if tuple(fused.shape) != (2 * inner, hidden) or tuple(down_w.shape) != (hidden, inner):
            return None
        if not (dense_gate_up_swiglu_applies(hidden, inner) and dense_down_residual_applies(hidden, inner)):
            return None
        if not hip_device(fused, down_w):
            return None
        return cls(fused.detach().contiguous(), down_w.detach().contiguous())

    def __call__(self, row: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
        activated = ops.dense_gate_up_swiglu(row.reshape(-1).contiguous(), self.fused_weight)
        return ops.dense_down_residual(activated, self.down_weight,
                                       residual.reshape(-1).to(torch.bfloat16).contiguous())


_STRATEGIES = (HipDenseMlp, DefaultMlp)


class Mlp(MlpStrategy):
    """The dense MLP a block declares: picks its binding once, then forwards every call."""

    def __init__(self, leaf, *, hidden: int, inner: int, activation: Activation = "silu",
                 reference: bool = False) -> None:
        self.strategy: MlpStrategy = resolve(
            (DefaultMlp,) if reference else _STRATEGIES, leaf, hidden=hidden, inner=inner,
            activation=activation,
        )

    def __call__(self, row: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
        return self.strategy(row, residual)

"""The routed down/combine primitive of a one-token step, `GateUp`'s sibling:
(act, chosen [n], weights [n], residual [hidden]) -> [hidden], each activation row
down-projected by its expert, routing-weighted, summed and residual-added.

Mirrors core/kernels/down_combine/__init__.py and kernel.py (`DownCombine`,
`DownCombineStrategy`, `Layout`).

- `HipNvfp4PackedDownCombine` (`omnia_moe_down_combine_nvfp4_shared`, csrc/moe_fp4.hip)
  serves what the reference's `Nvfp4PackedDownCombine` serves
  (core/kernels/down_combine/nvfp4_packed.py:196-270): an NVFP4 stack under the
  `interleaved` layout with a required NVFP4 shared expert (`QuantizedLinearLeaf`) of
  the same width, inner 512, hidden a multiple of 4, no bias, and both scale planes
  passing the halved plane's certificate (every odd byte of a group pair equal to the
  even one except flat pair 0, every byte below 128; shared/nvfp4/packed.py:150-162);
  any number of tokens, 1 to 31 routed slots. The shared stack runs on the last slot,
  unweighted, and the epilogue is bf16 at every step.
- `HipNvfp4DownCombine` (`omnia_moe_down_combine_nvfp4`, csrc/moe_fp4.hip) serves what
  the reference's `Nvfp4DownCombine` serves (core/kernels/down_combine/nvfp4.py:76-98): an
  NVFP4 stack under the `interleaved` layout, no bias or shared expert, hidden and inner
  multiples of 32 (inner up to 4096), at most 16 slots (more go to the Core chain). Per
  slot bf16(bf16(dot) * weight), the slot sum in fp32 in slot order, then the residual.
- `HipMxfp4DownCombine` (`omnia_moe_down_combine_mxfp4`, csrc/moe_fp4.hip) serves what
  the reference's `Mxfp4DownCombine` serves (core/kernels/down_combine/mxfp4.py:80-101):
  an MXFP4 stack under the `interleaved` layout with the per-row projection bias, no
  shared expert, hidden and inner multiples of 32 (inner up to 4096), at most 16 slots
  (more go to the Core chain). Per slot bf16(bf16(dot + bias) * weight), the slot sum in
  fp32 in slot order, then the residual add, in one dispatch.
- `HipAffineDownCombine` (`omnia_moe_down_combine_affine`, csrc/moe_affine.hip) serves
  what the reference's `AffineDownCombine` serves (core/kernels/down_combine/affine.py:
  97-178): an affine-quantized stack under the `interleaved` layout (the activation rows
  arrive activated), no bias, a shared expert on the last slot when it is an affine
  `QuantizedLinearLeaf`, inner a multiple of 32 up to 1536, at most 16 slots (more go to
  the Core chain). Per slot bf16(bf16(dot) * weight), the slot sum in fp32 in slot
  order, then the residual add, in one dispatch.
- `HipDenseDownCombine` (`omnia_moe_down_combine`, csrc/moe.hip) serves what the
  reference's `DenseDownCombine` serves (core/kernels/down_combine/dense.py:69-109): a
  dense bf16 stack [experts, hidden, inner] under the `blocked` layout (the pair block
  arrives un-activated and the SwiGLU runs inside the kernel), no bias, no shared
  expert, at most 16 experts per token. Its arithmetic is the dense binding's: the
  activation in fp32, bf16(dot * weight) per expert, then the expert sum and the
  residual add in bf16, all in one dispatch.
- `DefaultDownCombine` is the Core chain (core/kernels/down_combine/default.py:24-58): the
  activation in bf16 ops, the gathered matrices (dequantized for a quantized leaf) times
  the rows with an fp32 sum, the routing weights,
  the sum and the residual in torch ops. It accepts everything.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Literal, Protocol, runtime_checkable

import torch

from ...runtime import ops
from .._device import hip_device
from ..gate_up.routed import affine_leaf, mxfp4_applies, mxfp4_leaf, nvfp4_leaf
from ..leaf import QuantizedLinearLeaf, QuantizedSwitchLinearLeaf
from ..resolve import record_fallback, resolve

Layout = Literal["interleaved", "blocked"]
MAX_SLOTS = 16

__all__ = ["DefaultDownCombine", "DownCombine", "DownCombineStrategy", "HipAffineDownCombine",
           "HipDenseDownCombine", "HipMxfp4DownCombine", "HipNvfp4DownCombine", "HipNvfp4PackedDownCombine",
           "Layout", "affine_down_applies", "dense_down_applies", "packed_down_applies", "packed_plane_certified"]


@runtime_checkable
class DownCombineStrategy(Protocol):
    def __call__(self, act: torch.Tensor, chosen: torch.Tensor, weights: torch.Tensor,
                 residual: torch.Tensor) -> torch.Tensor: ...


def dense_down_applies(inner: int) -> bool:
    """The lane's slice of the activation stays in registers: inner / 8 vectors over 32
    lanes, at most 8 each."""
    return 0 < inner <= 2048 and inner % 8 == 0


def affine_down_applies(inner: int, group: int, bits: int) -> bool:
    """Eight lanes share a row, each taking at most six 32-value steps of it."""
    return (0 < inner <= 1536 and inner % 32 == 0 and group in ops.AFFINE_GROUPS
            and inner % group == 0 and bits in ops.AFFINE_BITS)


@dataclass(frozen=True)
class DefaultDownCombine(DownCombineStrategy):
    leaf: object
    bias: torch.Tensor | None
    shared: Callable[[torch.Tensor], torch.Tensor] | None
    layout: Layout

    @classmethod
    def build(cls, leaf, *, hidden, inner, bias, shared, layout) -> "DefaultDownCombine":
        return cls(leaf, bias, shared, layout)

    def __call__(self, act, chosen, weights, residual):
        rows = act.reshape(chosen.shape[0], -1)
        if self.layout == "blocked":
            gate, up = torch.chunk(rows, 2, dim=-1)
            rows = gate * torch.sigmoid(gate) * up
        routed = chosen if self.shared is None else chosen[:-1]
        k = routed.shape[0]
        matrices = self.leaf.matrices(routed)
        down = (matrices @ rows[:k].float()[..., None]).squeeze(-1).to(rows.dtype)
        if self.bias is not None:
            down = down + self.bias[routed.long()]
        out = (down * weights[:k, None]).sum(dim=0)
        if self.shared is not None:
            out = out + weights[-1] * self.shared(rows[-1][None]).reshape(-1)
        return out if residual is None else out + residual


@dataclass(frozen=True)
class HipDenseDownCombine(DownCombineStrategy):
    weight: torch.Tensor
    fallback: DefaultDownCombine

    @classmethod
    def build(cls, leaf, *, hidden, inner, bias, shared, layout) -> "HipDenseDownCombine | None":
        weight = leaf.weight
        if layout != "blocked" or bias is not None or shared is not None:
            return None
        if weight.dtype != torch.bfloat16 or weight.dim() != 3:
            return None
        if tuple(weight.shape[1:]) != (hidden, inner) or not dense_down_applies(inner):
            return None
        if not hip_device(weight):
            return None
        return cls(weight.contiguous(), DefaultDownCombine(leaf, bias, shared, layout))

    def __call__(self, act, chosen, weights, residual):
        k = chosen.numel()
        if k == 0 or k > MAX_SLOTS:  # one wave per expert in a workgroup
            record_fallback(self, self.fallback)
            return self.fallback(act, chosen, weights, residual)
        device = self.weight.device
        return ops.moe_down_combine(
            act.reshape(k, -1).to(torch.bfloat16).contiguous(), self.weight,
            chosen.to(device=device, dtype=torch.int32).contiguous().reshape(-1),
            weights.to(device=device, dtype=torch.float32).contiguous().reshape(-1),
            None if residual is None else residual.reshape(-1).to(torch.bfloat16).contiguous(),
        )


@dataclass(frozen=True)
class HipAffineDownCombine(DownCombineStrategy):
    leaf: "ops.AffineLeaf"
    shared: "ops.AffineLeaf | None"
    fallback: DefaultDownCombine

    @classmethod
    def build(cls, leaf, *, hidden, inner, bias, shared, layout) -> "HipAffineDownCombine | None":
        if layout != "interleaved" or bias is not None:
            return None
        if not isinstance(leaf, QuantizedSwitchLinearLeaf):
            return None
        if not affine_down_applies(inner, leaf.group_size, leaf.bits):
            return None
        view = affine_leaf(leaf, hidden, inner, stacked=True)
        if view is None:
            return None
        spare = None
        if shared is not None:
            if not isinstance(shared, QuantizedLinearLeaf) or not affine_down_applies(
                    inner, shared.group_size, shared.bits):
                return None
            spare = affine_leaf(shared, hidden, inner, stacked=False)
            if spare is None or spare.weight.device != view.weight.device:
                return None
        return cls(view, spare, DefaultDownCombine(leaf, bias, shared, layout))

    def __call__(self, act, chosen, weights, residual):
        slots = chosen.numel()
        if slots == 0 or slots > MAX_SLOTS:  # one wave per slot in a workgroup
            record_fallback(self, self.fallback)
            return self.fallback(act, chosen, weights, residual)
        device = self.leaf.weight.device
        return ops.moe_down_combine_affine(
            act.reshape(slots, -1).to(torch.bfloat16).contiguous(), self.leaf,
            chosen.to(device=device, dtype=torch.int32).contiguous().reshape(-1),
            weights.to(device=device, dtype=torch.float32).contiguous().reshape(-1),
            None if residual is None else residual.reshape(-1).to(torch.bfloat16).contiguous(),
            shared=self.shared,
        )


@dataclass(frozen=True)
class HipMxfp4DownCombine(DownCombineStrategy):
    leaf: "ops.Mxfp4Leaf"
    fallback: DefaultDownCombine

    @classmethod
    def build(cls, leaf, *, hidden, inner, bias, shared, layout) -> "HipMxfp4DownCombine | None":
        if layout != "interleaved" or bias is None or shared is not None:
            return None
        if not mxfp4_applies(hidden, inner) or inner > 4096:  # two 64-chunk steps per lane
            return None
        view = mxfp4_leaf(leaf, bias, hidden, inner)
        if view is None:
            return None
        return cls(view, DefaultDownCombine(leaf, bias, shared, layout))

    def __call__(self, act, chosen, weights, residual):
        slots = chosen.numel()
        if slots == 0 or slots > MAX_SLOTS:  # one wave per slot in a workgroup
            record_fallback(self, self.fallback)
            return self.fallback(act, chosen, weights, residual)
        device = self.leaf.weight.device
        return ops.moe_down_combine_mxfp4(
            act.reshape(slots, -1).to(torch.bfloat16).contiguous(), self.leaf,
            chosen.to(device=device, dtype=torch.int32).contiguous().reshape(-1),
            weights.to(device=device, dtype=torch.float32).contiguous().reshape(-1),
            None if residual is None else residual.reshape(-1).to(torch.bfloat16).contiguous(),
        )


@dataclass(frozen=True)
class HipNvfp4DownCombine(DownCombineStrategy):
    leaf: "ops.Nvfp4Leaf"
    fallback: DefaultDownCombine

    @classmethod
    def build(cls, leaf, *, hidden, inner, bias, shared, layout) -> "HipNvfp4DownCombine | None":
        if layout != "interleaved" or bias is not None or shared is not None:
            return None
        if not mxfp4_applies(hidden, inner) or inner > 4096:  # two 64-chunk steps per lane
            return None
        view = nvfp4_leaf(leaf, hidden, inner)
        if view is None:
            return None
        return cls(view, DefaultDownCombine(leaf, bias, shared, layout))

    def __call__(self, act, chosen, weights, residual):
        slots = chosen.numel()
        if slots == 0 or slots > MAX_SLOTS:  # one wave per slot in a workgroup
            record_fallback(self, self.fallback)
            return self.fallback(act, chosen, weights, residual)
        device = self.leaf.weight.device
        return ops.moe_down_combine_nvfp4(
            act.reshape(slots, -1).to(torch.bfloat16).contiguous(), self.leaf,
            chosen.to(device=device, dtype=torch.int32).contiguous().reshape(-1),
            weights.to(device=device, dtype=torch.float32).contiguous().reshape(-1),
            None if residual is None else residual.reshape(-1).to(torch.bfloat16).contiguous(),
        )


def packed_plane_certified(scales: torch.Tensor) -> bool:
    """Whether an e4m3 plane [..., in / 16] is one the reference's halved group-32 plane
    accepts (shared/nvfp4/packed.py:150-162): read as byte pairs, every odd byte equals its
    even partner except in flat pair 0 (the quantizer's first span), and no byte has its
    sign bit set."""
    if scales.dtype != torch.uint8 or scales.numel() == 0 or scales.shape[-1] % 2:
        return False
    pairs = scales.reshape(-1, 2)
    differ = pairs[1:, 0] != pairs[1:, 1]
    return not bool(differ.any()) and int(scales.max()) < 128


def packed_down_applies(hidden: int, inner: int, top_k: int | None = None) -> bool:
    """The reference's shape rule (nvfp4_packed.py:185-190): one 512-wide contraction,
    hidden a multiple of 4, 1 to 31 routed slots."""
    return hidden % 4 == 0 and hidden > 0 and inner == 512 and (top_k is None or 0 < top_k <= 31)


@dataclass(frozen=True)
class HipNvfp4PackedDownCombine(DownCombineStrategy):
    leaf: "ops.Nvfp4Leaf"
    shared: "ops.Nvfp4Leaf"

    @classmethod
    def build(cls, leaf, *, hidden, inner, bias, shared, layout) -> "HipNvfp4PackedDownCombine | None":
        if layout != "interleaved" or bias is not None or not packed_down_applies(hidden, inner):
            return None
        view = nvfp4_leaf(leaf, hidden, inner)
        if view is None:
            return None
        if (not isinstance(shared, QuantizedLinearLeaf) or shared.mode != "nvfp4" or shared.biases is not None
                or shared.bits != 4 or shared.group_size != 16):
            return None
        shared_view = ops.Nvfp4Leaf(shared.weight[None], shared.scales[None], None)
        try:
            shared_view.check(hidden, inner, "nvfp4 shared leaf")
        except ValueError:
            return None
        if not all(hip_device(t) for t in shared_view.tensors()):
            return None
        if not (packed_plane_certified(leaf.scales) and packed_plane_certified(shared.scales)):
            return None
        return cls(view, shared_view)

    def __call__(self, act, chosen, weights, residual):
        """act [..., top_k + 1, inner] (the shared slot last), chosen and weights
        [..., top_k + 1] (the last entries unread), residual [..., hidden]."""
        hidden = residual.shape[-1]
        tokens = residual.numel() // hidden
        slots = chosen.shape[-1]
        if not packed_down_applies(hidden, self.leaf.features, slots - 1):
            raise ValueError(f"packed NVFP4 down/combine: {slots - 1} routed slots, expected 1 to 31")
        device = self.leaf.weight.device
        out = ops.moe_down_combine_nvfp4_shared(
            act.reshape(tokens, slots, -1).to(torch.bfloat16).contiguous(), self.leaf, self.shared,
            chosen.reshape(tokens, slots)[:, :-1].to(device=device, dtype=torch.int32).contiguous(),
            weights.reshape(tokens, slots)[:, :-1].to(device=device, dtype=torch.float32).contiguous(),
            residual.reshape(tokens, hidden).to(torch.bfloat16).contiguous(),
        )
        return out.reshape(residual.shape)


_STRATEGIES = (HipNvfp4PackedDownCombine, HipNvfp4DownCombine, HipMxfp4DownCombine, HipAffineDownCombine,
               HipDenseDownCombine, DefaultDownCombine)


class DownCombine(DownCombineStrategy):
    """The routed down projection a block declares: picks its binding once, then forwards."""

    def __init__(self, leaf, *, hidden: int, inner: int, bias: torch.Tensor | None = None,
                 shared=None, layout: Layout = "interleaved", reference: bool = False) -> None:
        self.strategy: DownCombineStrategy = resolve(
            (DefaultDownCombine,) if reference else _STRATEGIES, leaf, hidden=hidden,
            inner=inner, bias=bias, shared=shared, layout=layout,
        )

    def __call__(self, act, chosen, weights, residual):
        return self.strategy(act, chosen, weights, residual)

"""The routed gate/up primitive of a one-token step: (row [hidden], chosen [k]) ->
[k, inner] (the activation) or [k, 2 * inner] (the un-activated pair block, `blocked`).

Mirrors core/kernels/gate_up/__init__.py and kernel.py (`GateUp`, `GateUpStrategy`,
`Layout`, `OrdinalRouting`): a block declares the expert leaf and the epilogue
(activation, clamp, projection bias, layout, ordinal routing, a shared expert), and the
first strategy whose `build` accepts the declaration serves it.

- `HipMxfp4GateUp` (`omnia_moe_gate_up_mxfp4`, csrc/moe_fp4.hip) serves what the
  reference's `Mxfp4GateUp` serves (core/kernels/gate_up/mxfp4.py:82-111): an MXFP4 stack
  (`QuantizedSwitchLinearLeaf` mode "mxfp4") under the `interleaved` layout, swiglu_oai
  with its clamp and the per-row projection bias, no ordinal routing or shared expert,
  hidden and inner multiples of 32 (hidden up to 16384).
- `HipNvfp4GateUp` (`omnia_moe_gate_up_nvfp4`, csrc/moe_fp4.hip) serves what the
  reference's `Nvfp4GateUp` serves (core/kernels/gate_up/nvfp4.py:79-110): an NVFP4 stack
  (mode "nvfp4", e4m3 scales per 16) under the `interleaved` layout, silu without clamp,
  bias or shared expert; hidden and inner multiples of 32 (the reference's 16: the others
  go to the Core chain), hidden up to 16384. With an `OrdinalRouting` declaration it
  serves what `Nvfp4PackedGateUp` serves (core/kernels/gate_up/nvfp4_packed.py:286-321)
  through `omnia_moe_gate_up_nvfp4_ordinal`, which ranks uint32 ordinal keys in the
  kernel (up to 1024 experts; other key types go to the Core chain).
- `HipAffineGateUp` (`omnia_moe_gate_up_affine`, csrc/moe_affine.hip) serves what the
  reference's `AffineGateUp` serves (core/kernels/gate_up/affine.py:105-191): an
  affine-quantized stack (`QuantizedSwitchLinearLeaf`, 2, 3, 4, 5, 6 or 8 bits, groups of
  32, 64 or 128) under the `interleaved` layout, silu with the optional clamp, no bias
  or ordinal routing, and a shared expert on the last slot when it is an affine
  `QuantizedLinearLeaf` of its own width and group.
- `HipDenseGateUp` (`omnia_moe_gate_up`, csrc/moe.hip) serves what the reference's
  `DenseGateUp` serves (core/kernels/gate_up/dense.py:75-119): a dense bf16 stack
  [experts, 2 * inner, hidden], the `blocked` layout (gate and up block-concatenated,
  handed on un-activated), silu, no clamp, bias, routing or shared expert.
- `DefaultGateUp` is the Core chain (core/kernels/gate_up/default.py:31-81): the gathered
  matrices (dequantized for a quantized leaf) times the row with an fp32 sum, then the
  declared epilogue in bf16 ops. It accepts everything.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Literal, Protocol, runtime_checkable

import torch

from ...runtime import ops
from .._device import hip_device
from ..leaf import QuantizedLinearLeaf, QuantizedSwitchLinearLeaf
from ..resolve import record_fallback, resolve

Activation = Literal["silu", "swiglu_oai"]
Layout = Literal["interleaved", "blocked"]


@dataclass(frozen=True)
class OrdinalRouting:
    """The second argument carries the router's ordinal keys [experts] (ascending =
    better); the strategy keeps the `top_k` best, equal keys to the lower index
    (core/kernels/gate_up/kernel.py:23-36)."""

    top_k: int

    def indices(self, keys: torch.Tensor) -> torch.Tensor:
        return torch.sort(keys.to(torch.int64), stable=True).indices[: self.top_k].to(torch.int32)


@runtime_checkable
class GateUpStrategy(Protocol):
    def __call__(self, row: torch.Tensor, chosen: torch.Tensor) -> torch.Tensor: ...


def dense_gate_up_applies(hidden: int) -> bool:
    """A row is hidden / 8 16-byte vectors, at most 16 per lane."""
    return 0 < hidden <= 8192 and hidden % 8 == 0


def affine_gate_up_applies(hidden: int, group: int, bits: int) -> bool:
    """32 values per lane step, inside one quantization group."""
    return (0 < hidden <= 16384 and hidden % 32 == 0 and group in ops.AFFINE_GROUPS
            and hidden % group == 0 and bits in ops.AFFINE_BITS)


def affine_leaf(leaf, rows: int, features: int, stacked: bool) -> "ops.AffineLeaf | None":
    """The kernels' view of an affine leaf whose tensors they can read as they are, or None."""
    wanted = QuantizedSwitchLinearLeaf if stacked else QuantizedLinearLeaf
    if not isinstance(leaf, wanted) or leaf.mode != "affine" or leaf.biases is None:
        return None
    if leaf.bits not in ops.AFFINE_BITS or leaf.group_size not in ops.AFFINE_GROUPS:
        return None
    if features % leaf.group_size != 0:
        return None
    view = ops.AffineLeaf(leaf.weight, leaf.scales, leaf.biases, leaf.bits, leaf.group_size)
    try:
        view.check(rows, features, stacked, "affine leaf")
    except ValueError:
        return None
    if not all(hip_device(t) for t in view.tensors()):
        return None
    return view


def mxfp4_applies(hidden: int, inner: int) -> bool:
    """Both contractions cover whole 32-value e8m0 groups (core/kernels/shared/mxfp4.py:
    35-38)."""
    return hidden > 0 and inner > 0 and hidden % 32 == 0 and inner % 32 == 0


def mxfp4_leaf(leaf, bias, rows: int, features: int) -> "ops.Mxfp4Leaf | None":
    """The kernels' view of an MXFP4 stack and its projection bias [experts, rows], or None."""
    if not isinstance(leaf, QuantizedSwitchLinearLeaf) or leaf.mode != "mxfp4":
        return None
    if leaf.biases is not None or leaf.bits != 4 or leaf.group_size != 32:
        return None
    if bias is None or bias.dtype != torch.bfloat16:
        return None
    view = ops.Mxfp4Leaf(leaf.weight, leaf.scales, bias.contiguous())
    try:
        view.check(rows, features, "mxfp4 leaf")
    except ValueError:
        return None
    if not all(hip_device(t) for t in view.tensors()):
        return None
    return view


def nvfp4_leaf(leaf, rows: int, features: int) -> "ops.Nvfp4Leaf | None":
    """The kernels' view of an NVFP4 stack [experts, rows, ...], or None."""
    if not isinstance(leaf, QuantizedSwitchLinearLeaf) or leaf.mode != "nvfp4":
        return None
    if leaf.biases is not None or leaf.bits != 4 or leaf.group_size != 16:
        return None
    view = ops.Nvfp4Leaf(leaf.weight, leaf.scales, None)
    try:
        view.check(rows, features, "nvfp4 leaf")
    except ValueError:
        return None
    if not all(hip_device(t) for t in view.tensors()):
        return None
    return view


@dataclass(frozen=True)
class DefaultGateUp(GateUpStrategy):
    leaf: object
    activation: Activation
    limit: float | None
    bias: torch.Tensor | None
    layout: Layout
    routing: OrdinalRouting | None
    shared: Callable[[torch.Tensor], torch.Tensor] | None

    @classmethod
    def build(cls, leaf, *, hidden, inner, activation, limit, bias, layout, routing,
              shared) -> "DefaultGateUp":
        assert shared is None or routing is None
        return cls(leaf, activation, limit, bias, layout, routing, shared)

    def __call__(self, row: torch.Tensor, chosen: torch.Tensor) -> torch.Tensor:
        if self.routing is not None:
            chosen = self.routing.indices(chosen)
        routed = chosen if self.shared is None else chosen[:-1]
        matrices = self.leaf.matrices(routed)
        fused = (matrices @ row.reshape(-1).float()).to(row.dtype)
        if self.bias is not None:
            fused = fused + self.bias[routed.long()]
        if self.shared is not None:
            fused = torch.cat([fused, self.shared(row.reshape(1, -1)).reshape(1, -1)], dim=0)
        if self.layout == "blocked":
            return fused
        pairs = fused.reshape(fused.shape[0], -1, 2)
        gate, up = pairs[..., 0], pairs[..., 1]
        if self.activation == "swiglu_oai":
            assert self.limit is not None
            gate = torch.clamp(gate, max=self.limit)
            up = torch.clamp(up, -self.limit, self.limit)
            return gate * torch.sigmoid(1.702 * gate) * (up + 1)
        if self.limit is not None:
            gate = torch.clamp(gate, max=self.limit)
            up = torch.clamp(up, -self.limit, self.limit)
        return gate * torch.sigmoid(gate) * up


@dataclass(frozen=True)
class HipDenseGateUp(GateUpStrategy):
    weight: torch.Tensor

    @classmethod
    def build(cls, leaf, *, hidden, inner, activation, limit, bias, layout, routing,
              shared) -> "HipDenseGateUp | None":
        weight = leaf.weight
        if shared is not None or routing is not None or bias is not None or limit is not None:
            return None
        if layout != "blocked" or activation != "silu":
            return None
        if weight.dtype != torch.bfloat16 or weight.dim() != 3:
            return None
        if tuple(weight.shape[1:]) != (2 * inner, hidden) or not dense_gate_up_applies(hidden):
            return None
        if not hip_device(weight):
            return None
        return cls(weight.contiguous())

    def __call__(self, row: torch.Tensor, chosen: torch.Tensor) -> torch.Tensor:
        ids = chosen.to(device=self.weight.device, dtype=torch.int32).contiguous().reshape(-1)
        return ops.moe_gate_up(row.reshape(-1).contiguous(), self.weight, ids)


@dataclass(frozen=True)
class HipAffineGateUp(GateUpStrategy):
    leaf: "ops.AffineLeaf"
    limit: float | None
    shared: "ops.AffineLeaf | None"

    @classmethod
    def build(cls, leaf, *, hidden, inner, activation, limit, bias, layout, routing,
              shared) -> "HipAffineGateUp | None":
        if layout != "interleaved" or routing is not None:
            return None
        if activation != "silu" or bias is not None or (limit is not None and not limit >= 0):
            return None
        if not isinstance(leaf, QuantizedSwitchLinearLeaf):
            return None
        if not affine_gate_up_applies(hidden, leaf.group_size, leaf.bits):
            return None
        view = affine_leaf(leaf, 2 * inner, hidden, stacked=True)
        if view is None:
            return None
        spare = None
        if shared is not None:
            if not isinstance(shared, QuantizedLinearLeaf):
                return None
            spare = affine_leaf(shared, 2 * inner, hidden, stacked=False)
            if spare is None or spare.weight.device != view.weight.device:
                return None
        return cls(view, limit, spare)

    def __call__(self, row: torch.Tensor, chosen: torch.Tensor) -> torch.Tensor:
        ids = chosen.to(device=self.leaf.weight.device, dtype=torch.int32).contiguous().reshape(-1)
        return ops.moe_gate_up_affine(row.reshape(-1).contiguous(), self.leaf, ids,
                                      limit=self.limit, shared=self.shared)


@dataclass(frozen=True)
class HipMxfp4GateUp(GateUpStrategy):
    leaf: "ops.Mxfp4Leaf"
    limit: float

    @classmethod
    def build(cls, leaf, *, hidden, inner, activation, limit, bias, layout, routing,
              shared) -> "HipMxfp4GateUp | None":
        # The spare slot is the affine kernel's: a shared expert beside this stack has no
        # kernel here, as in the reference.
        if shared is not None or layout != "interleaved" or routing is not None:
            return None
        if activation != "swiglu_oai" or limit is None or not limit >= 0 or bias is None:
            return None
        if not mxfp4_applies(hidden, inner) or hidden > 16384:
            return None
        view = mxfp4_leaf(leaf, bias, 2 * inner, hidden)
        return None if view is None else cls(view, float(limit))

    def __call__(self, row: torch.Tensor, chosen: torch.Tensor) -> torch.Tensor:
        ids = chosen.to(device=self.leaf.weight.device, dtype=torch.int32).contiguous().reshape(-1)
        return ops.moe_gate_up_mxfp4(row.reshape(-1).contiguous(), self.leaf, ids, limit=self.limit)


@dataclass(frozen=True)
class HipNvfp4GateUp(GateUpStrategy):
    leaf: "ops.Nvfp4Leaf"
    routing: OrdinalRouting | None
    fallback: "DefaultGateUp"

    @classmethod
    def build(cls, leaf, *, hidden, inner, activation, limit, bias, layout, routing,
              shared) -> "HipNvfp4GateUp | None":
        if shared is not None or layout != "interleaved":
            return None
        # The kernel carries neither clamp nor projection bias, as the reference's.
        if activation != "silu" or limit is not None or bias is not None:
            return None
        if not mxfp4_applies(hidden, inner) or hidden > 16384:
            return None
        view = nvfp4_leaf(leaf, 2 * inner, hidden)
        if view is None:
            return None
        if routing is not None and not 0 < routing.top_k <= view.weight.shape[0] <= 1024:
            return None
        fallback = DefaultGateUp.build(leaf, hidden=hidden, inner=inner, activation=activation,
                                       limit=limit, bias=bias, layout=layout, routing=routing,
                                       shared=shared)
        return cls(view, routing, fallback)

    def __call__(self, row: torch.Tensor, chosen: torch.Tensor) -> torch.Tensor:
        x = row.reshape(-1).contiguous()
        if self.routing is not None:
            # Ordinal keys are uint32 (the router's ordinals); the kernel ranks them in place
            # of the sort (core/kernels/gate_up/nvfp4_packed.py:1-13).
            if chosen.dtype != torch.uint32:
                record_fallback(self, self.fallback)
                return self.fallback(row, chosen)
            keys = chosen.to(device=self.leaf.weight.device).contiguous().reshape(-1)
            return ops.moe_gate_up_nvfp4_ordinal(x, self.leaf, keys, self.routing.top_k)
        ids = chosen.to(device=self.leaf.weight.device, dtype=torch.int32).contiguous().reshape(-1)
        return ops.moe_gate_up_nvfp4(x, self.leaf, ids)


_STRATEGIES = (HipNvfp4GateUp, HipMxfp4GateUp, HipAffineGateUp, HipDenseGateUp, DefaultGateUp)


class GateUp(GateUpStrategy):
    """The routed gate/up a block declares: picks its binding once, then forwards."""

    def __init__(self, leaf, *, hidden: int, inner: int, activation: Activation = "silu",
                 limit: float | None = None, bias: torch.Tensor | None = None,
                 layout: Layout = "interleaved", routing: OrdinalRouting | None = None,
                 shared=None, reference: bool = False) -> None:
        self.strategy: GateUpStrategy = resolve(
            (DefaultGateUp,) if reference else _STRATEGIES, leaf, hidden=hidden, inner=inner,
            activation=activation, limit=limit, bias=bias, layout=layout, routing=routing,
            shared=shared,
        )

    def __call__(self, row: torch.Tensor, chosen: torch.Tensor) -> torch.Tensor:
        return self.strategy(row, chosen)

"""Leaves: the declaration objects the facades read.

The reference's blocks hand `nn.RMSNorm` leaves (`.weight`, `.eps`) to the residual-join
facades, `SwitchLinear` stacks to the routed expert facades and `SwiGLU` modules to the
dense MLP facade; these are the minimal torch stand-ins.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

import torch


@dataclass
class RMSNormLeaf:
    weight: torch.Tensor
    eps: float = 1e-6


@dataclass
class SwitchLinearLeaf:
    """A stack of expert matrices, one per row: weight [experts, out, in], the layout of
    the reference's `SwitchLinear` leaf (core/layers.py:140-154)."""

    weight: torch.Tensor

    def matrices(self, index: torch.Tensor) -> torch.Tensor:
        """The indexed experts' matrices as float32 [k, out, in]."""
        return self.weight[index.long()].float()


def unpack_words(words: torch.Tensor, bits: int) -> torch.Tensor:
    """32-bit words [..., n] -> int64 values [..., n * 32 / bits]: each row one
    little-endian bit stream, value j at bit j * bits (core/kernels/shared/affine.py:9-58
    decodes the same bytes)."""
    w = words.to(torch.int64) & 0xFFFFFFFF
    count = w.shape[-1] * 32 // bits
    bit = torch.arange(count, device=w.device) * bits
    word, shift = bit // 32, bit % 32
    padded = torch.cat([w, torch.zeros_like(w[..., :1])], dim=-1)
    window = w[..., word] | (padded[..., word + 1] << 32)
    return (window >> shift) & ((1 << bits) - 1)


def affine_dequantize(words: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                      group_size: int, bits: int) -> torch.Tensor:
    """scale * q + bias per group, float32 [..., out, in]."""
    q = unpack_words(words, bits).float()
    s = scales.float().repeat_interleave(group_size, dim=-1)
    b = biases.float().repeat_interleave(group_size, dim=-1)
    return s * q + b


@dataclass
class QuantizedSwitchLinearLeaf:
    """An affine-quantized expert stack, the reference's `QuantizedSwitchLinear` leaf
    (core/layers.py:164-197): weight [experts, out, in * bits / 32] 32-bit words (int32 or
    uint32), scales and biases [experts, out, in / group_size] bf16. Only mode "affine"
    carries biases; other modes are declared but decoded by nothing here."""

    weight: torch.Tensor
    scales: torch.Tensor
    biases: torch.Tensor | None
    group_size: int
    bits: int
    mode: str = "affine"

    def matrices(self, index: torch.Tensor) -> torch.Tensor:
        """The indexed experts' dequantized matrices as float32 [k, out, in]."""
        if self.mode != "affine" or self.biases is None:
            raise NotImplementedError(f"no decoder for quantization mode {self.mode!r}")
        i = index.long()
        return affine_dequantize(self.weight[i], self.scales[i], self.biases[i], self.group_size, self.bits)


@dataclass
class QuantizedLinearLeaf:
    """One affine-quantized matrix, `nn.QuantizedLinear` (weight [out, in * bits / 32],
    scales and biases [out, in / group_size]); called as the layer, x [..., in] ->
    [..., out] with an fp32 sum rounded to x's dtype, as mx.quantized_matmul does."""

    weight: torch.Tensor
    scales: torch.Tensor
    biases: torch.Tensor | None
    group_size: int
    bits: int
    mode: str = "affine"

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        if self.mode != "affine" or self.biases is None:
            raise NotImplementedError(f"no decoder for quantization mode {self.mode!r}")
        w = affine_dequantize(self.weight, self.scales, self.biases, self.group_size, self.bits)
        return (x.float() @ w.T).to(x.dtype)


def swish(x: torch.Tensor) -> torch.Tensor:
    return x * torch.sigmoid(x)


class SwiGLU(torch.nn.Module):
    """gate||up concatenated on the output axis (gate rows first) and split back by slice,
    then the down projection: core/layers.py:253-272. The projections are bias-free
    `nn.Linear` layers, as there; `activation` is the only thing architectures vary."""

    def __init__(self, hidden: int, inner: int,
                 activation: Callable[[torch.Tensor], torch.Tensor] = swish) -> None:
        super().__init__()
        self.inner = inner
        self.gate_up_proj = torch.nn.Linear(hidden, 2 * inner, bias=False)
        self.down_proj = torch.nn.Linear(inner, hidden, bias=False)
        self._activation = activation

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gate, up = torch.split(self.gate_up_proj(x), [self.inner, self.inner], dim=-1)
        return self.down_proj(self._activation(gate) * up)

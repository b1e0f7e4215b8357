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


E2M1 = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)


def mxfp4_dequantize(words: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """e2m1 codes (4-bit, the low nibble of each byte first) times their 32-value group's
    e8m0 factor, the fp32 whose exponent field is the scale byte (2^(byte - 127), 0 for
    byte 0): float32 [..., out, in] (core/kernels/shared/mxfp4.py:8-32 decodes the same
    bytes)."""
    table = torch.tensor(E2M1, dtype=torch.float32, device=words.device)
    values = table[unpack_words(words, 4)]
    factors = (scales.to(torch.int32) << 23).contiguous().view(torch.float32)
    return values * factors.repeat_interleave(32, dim=-1)


def e4m3_values(scales: torch.Tensor) -> torch.Tensor:
    """e4m3 bytes -> float32 as mlx decodes them: the magnitude bits placed in a half's
    exponent and top mantissa bits and scaled by 2^8, the sign from bit 7, so 0x7F is 480
    (core/kernels/shared/nvfp4/qmoe.py:22-37)."""
    b = scales.to(torch.int32)
    half = ((b & 0x7F) << 7).to(torch.int16).view(torch.float16).float() * 256.0
    return torch.where((b & 0x80) != 0, -half, half)


def nvfp4_dequantize(words: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """e2m1 codes times their 16-value group's e4m3 factor: float32 [..., out, in]."""
    table = torch.tensor(E2M1, dtype=torch.float32, device=words.device)
    values = table[unpack_words(words, 4)]
    return values * e4m3_values(scales.contiguous()).repeat_interleave(16, dim=-1)


def dequantize(leaf, index: torch.Tensor | None = None) -> torch.Tensor:
    """A quantized leaf's matrices (the indexed experts' for a stack) as float32."""
    pick = (lambda t: t) if index is None else (lambda t: t[index.long()])
    if leaf.mode == "affine" and leaf.biases is not None:
        return affine_dequantize(pick(leaf.weight), pick(leaf.scales), pick(leaf.biases),
                                 leaf.group_size, leaf.bits)
    if leaf.mode == "mxfp4" and leaf.biases is None and leaf.bits == 4 and leaf.group_size == 32:
        return mxfp4_dequantize(pick(leaf.weight), pick(leaf.scales))
    if leaf.mode == "nvfp4" and leaf.biases is None and leaf.bits == 4 and leaf.group_size == 16:
        return nvfp4_dequantize(pick(leaf.weight), pick(leaf.scales))
    raise NotImplementedError(f"no decoder for quantization mode {leaf.mode!r}")


@dataclass
class QuantizedSwitchLinearLeaf:
    """A quantized expert stack, the reference's `QuantizedSwitchLinear` leaf
    (core/layers.py:164-197): weight [experts, out, in * bits / 32] 32-bit words (int32 or
    uint32) and scales [experts, out, in / group_size]. Mode "affine": bf16 scales and
    biases, 2-8 bits. Mode "mxfp4": 4 bits, groups of 32, uint8 e8m0 scales, no biases.
    Mode "nvfp4": 4 bits, groups of 16, uint8 e4m3 scales, no biases. Other modes are
    declared but decoded by nothing here."""

    weight: torch.Tensor
    scales: torch.Tensor
    biases: torch.Tensor | None
    group_size: int
    bits: int
    mode: str = "affine"

    def matrices(self, index: torch.Tensor) -> torch.Tensor:
        """The indexed experts' dequantized matrices as float32 [k, out, in]."""
        return dequantize(self, index)


@dataclass
class QuantizedLinearLeaf:
    """One quantized matrix, `nn.QuantizedLinear` (weight [out, in * bits / 32], scales
    [out, in / group_size], biases in mode "affine"); called as the layer, x [..., in] ->
    [..., out] with an fp32 sum rounded to x's dtype, as mx.quantized_matmul does."""

    weight: torch.Tensor
    scales: torch.Tensor
    biases: torch.Tensor | None
    group_size: int
    bits: int
    mode: str = "affine"

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        return (x.float() @ dequantize(self).T).to(x.dtype)


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

"""Embedding gather + atlas rows in one HIP dispatch (`omnia_embed_atlas`,
csrc/embed_atlas.hip).

Serves what core/kernels/embed/atlas.py:95-109 (`AtlasEmbed.build`) serves — a bf16
embedding and fp32 atlases whose widths are multiples of 4 — for any number of tokens.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ...runtime import ops
from .._device import hip_device
from .kernel import EmbedStrategy, segment_length


def applies(hidden: int, full_width: int, sliding_width: int, *, dtype: torch.dtype) -> bool:
    """Every copy moves 16-byte vectors with no tail: hidden a multiple of 8 (bf16), both
    atlas widths multiples of 4 (fp32); a hidden row fits 16 vectors per lane."""
    return (
        dtype == torch.bfloat16
        and hidden % 8 == 0
        and 0 < hidden <= 8192
        and full_width % 4 == 0
        and sliding_width % 4 == 0
    )


@dataclass(frozen=True)
class HipEmbed(EmbedStrategy):
    embedding: torch.Tensor
    full_atlas: torch.Tensor
    sliding_atlas: torch.Tensor

    @classmethod
    def build(cls, embedding, *, full_atlas, sliding_atlas) -> "HipEmbed | None":
        if full_atlas.dtype != torch.float32 or sliding_atlas.dtype != torch.float32:
            return None
        if not applies(embedding.shape[-1], full_atlas.shape[-1], sliding_atlas.shape[-1],
                       dtype=embedding.dtype):
            return None
        if not hip_device(embedding, full_atlas, sliding_atlas):
            return None
        return cls(embedding.contiguous(), full_atlas.contiguous(), sliding_atlas.contiguous())

    def __call__(self, tokens: torch.Tensor, position: int):
        length = segment_length(tokens)
        ids = tokens.to(device=self.embedding.device, dtype=torch.int32).contiguous()
        hidden, full, sliding = ops.embed_atlas(
            ids, self.embedding, self.full_atlas, self.sliding_atlas,
            position=position, n_positions=length,
        )
        if tokens.numel() == 1:
            return hidden.reshape(-1), full.reshape(-1), sliding.reshape(-1)
        return hidden, full, sliding

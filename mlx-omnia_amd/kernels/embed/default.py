"""The Core embed strategy: three gathers (core/kernels/embed/default.py:19-42).

`build` accepts every embedding and atlas pair, so it registers last and makes the facade
total.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .kernel import EmbedStrategy, segment_length


@dataclass(frozen=True)
class DefaultEmbed(EmbedStrategy):
    embedding: torch.Tensor
    full_atlas: torch.Tensor
    sliding_atlas: torch.Tensor

    @classmethod
    def build(cls, embedding, *, full_atlas, sliding_atlas) -> "DefaultEmbed":
        return cls(embedding, full_atlas, sliding_atlas)

    def __call__(self, tokens: torch.Tensor, position: int):
        length = segment_length(tokens)
        rows = slice(position, position + length)
        full = self.full_atlas.reshape(-1, self.full_atlas.shape[-1])[rows]
        sliding = self.sliding_atlas.reshape(-1, self.sliding_atlas.shape[-1])[rows]
        if tokens.numel() == 1:
            return self.embedding[tokens.reshape(-1)].reshape(-1), full.reshape(-1), sliding.reshape(-1)
        return self.embedding[tokens.long()], full, sliding

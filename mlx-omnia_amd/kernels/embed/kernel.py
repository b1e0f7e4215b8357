"""The embed primitive's contract (core/kernels/embed/kernel.py:1-31).

`(tokens, position) -> (hidden, full_angles, sliding_angles)`: the tokens' embedding rows
plus the rows of two position-indexed RoPE angle atlases. Three pure copies, no
arithmetic: every strategy is bit-identical to the stock gathers. The reference serves
one decoded token; the facade here also serves a segment, tokens [..., L] sharing the
positions position .. position+L-1. A single token keeps the reference's shapes:
hidden [H], full [FW], sliding [SW]; a segment gives [..., L, H], [L, FW], [L, SW].
"""

from __future__ import annotations

from typing import Protocol, runtime_checkable

import torch


@runtime_checkable
class EmbedStrategy(Protocol):
    def __call__(
        self, tokens: torch.Tensor, position: int
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]: ...


def segment_length(tokens: torch.Tensor) -> int:
    return 1 if tokens.numel() == 1 else tokens.shape[-1]

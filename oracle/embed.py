"""Embedding gather + RoPE atlas rows (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

Pure copies, restating core/kernels/embed/default.py:35-42 (`embedding[tokens]`, and
row `position` of each atlas flattened to [positions, width]) for a segment: token i's
row, and the atlas rows at positions position .. position+n-1. An id outside the table
gives a zero row (the HIP kernel's documented behaviour; the reference asserts instead).
"""

from __future__ import annotations

import numpy as np


def embed_atlas(tokens: np.ndarray, embedding: np.ndarray, full_atlas, sliding_atlas,
                position: int, n_positions: int):
    """tokens int32 [...]; embedding uint16 [vocab, H]; atlases float32 [..., rows, W]."""
    ids = np.asarray(tokens).astype(np.int64)
    valid = (ids >= 0) & (ids < embedding.shape[0])
    hidden = np.where(valid[..., None], embedding[np.where(valid, ids, 0)], np.uint16(0))
    rows = slice(position, position + n_positions)
    full = None if full_atlas is None else full_atlas.reshape(-1, full_atlas.shape[-1])[rows]
    sliding = None if sliding_atlas is None else sliding_atlas.reshape(-1, sliding_atlas.shape[-1])[rows]
    return hidden.astype(np.uint16), full, sliding

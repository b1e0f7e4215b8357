"""The two KV caches the fused decode step writes into, reduced to what the step needs.

Mirrors core/cache/kv.py: `FixedKVCache` (:131-275), a fixed-capacity buffer whose
position lives on the device so a captured step replays it, and `RingKVCache`
(:326-420), a sliding window of `window` rows written at `position % window`. Buffers are
[1, kv_heads, rows, head_dim] (the reference's layout). `offset` is the host's copy of the
position; `position` the device one, advanced together by `advance`.
"""

from __future__ import annotations

import torch


class FixedKVCache:
    def __init__(self, keys: torch.Tensor, values: torch.Tensor, position: int = 0) -> None:
        assert keys.shape == values.shape and keys.dim() == 4 and keys.shape[0] == 1
        self.keys, self.values = keys, values
        self.offset = position
        self.position = torch.tensor([position], dtype=torch.int32, device=keys.device)
        # The last position a captured step's replays may reach (None: not declared). A
        # fixed cache is bounded by its capacity; a ring's position has no bound of its
        # own, so a step over it is captured only after this is declared.
        self.replay_limit: int | None = None

    @classmethod
    def empty(cls, kv_heads: int, capacity: int, head_dim: int, *, dtype=torch.bfloat16,
              device=None) -> "FixedKVCache":
        shape = (1, kv_heads, capacity, head_dim)
        return cls(torch.zeros(shape, dtype=dtype, device=device),
                   torch.zeros(shape, dtype=dtype, device=device))

    @property
    def capacity(self) -> int:
        return self.keys.shape[2]

    @property
    def window(self) -> int:
        return 0

    def write_index(self) -> int:
        return self.offset

    def valid_rows(self) -> int:
        """Rows holding data: [0, offset)."""
        return min(self.offset, self.capacity)

    def fetch(self) -> tuple[torch.Tensor, torch.Tensor]:
        return self.keys, self.values

    def advance(self, rows: int = 1) -> None:
        """Account for rows a reader wrote into the buffer itself (kv.py:167-169)."""
        self.offset += rows
        self.position += rows

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        """Append [1, kv_heads, T, D] rows at the position; the rows written so far."""
        length = keys.shape[2]
        if self.offset + length > self.capacity:
            raise ValueError(f"cache of {self.capacity} rows cannot take row {self.offset + length - 1}")
        self.keys[:, :, self.offset : self.offset + length] = keys
        self.values[:, :, self.offset : self.offset + length] = values
        self.advance(length)
        return self.keys[:, :, : self.offset], self.values[:, :, : self.offset]


class RingKVCache(FixedKVCache):
    def __init__(self, keys: torch.Tensor, values: torch.Tensor, position: int = 0) -> None:
        super().__init__(keys, values, position)

    @classmethod
    def empty(cls, kv_heads: int, window: int, head_dim: int, *, dtype=torch.bfloat16,
              device=None) -> "RingKVCache":
        shape = (1, kv_heads, window, head_dim)
        return cls(torch.zeros(shape, dtype=dtype, device=device),
                   torch.zeros(shape, dtype=dtype, device=device))

    @property
    def window(self) -> int:
        return self.keys.shape[2]

    def write_index(self) -> int:
        return self.offset % self.window

    def valid_rows(self) -> int:
        """Slots written so far: the first min(offset, window) (kv.py:383-398)."""
        return min(self.offset, self.window)

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        """One row at a time, at position % window (kv.py:400-412); the filled slots."""
        assert keys.shape[2] == 1, "a ring appends one row at a time"
        index = self.write_index()
        self.keys[:, :, index : index + 1] = keys
        self.values[:, :, index : index + 1] = values
        self.advance(1)
        rows = self.valid_rows()
        return self.keys[:, :, :rows], self.values[:, :, :rows]


class KVCache:
    """A growing buffer [1, kv_heads, capacity, head_dim] for keys and one for values, the
    reference's `KVCache` (core/cache/kv.py:18-71): rows are appended at `offset`, and the
    buffers grow in blocks of 256 rows (`reserve`, kv.py:309-323), the old rows copied
    into the new ones. A sliding layer keeps every row too: its mask, not the cache,
    drops the old ones. `update_and_fetch` returns the rows written so far as views of
    the buffers, so the head stride is the capacity's."""

    BLOCK = 256

    def __init__(self, window: int | None = None) -> None:
        self.window = window
        self.offset = 0
        self.keys: torch.Tensor | None = None
        self.values: torch.Tensor | None = None

    @property
    def capacity(self) -> int:
        return 0 if self.keys is None else self.keys.shape[2]

    @classmethod
    def _reserve(cls, buffer: torch.Tensor | None, needed: int, like: torch.Tensor) -> torch.Tensor:
        if buffer is not None and buffer.shape[2] >= needed:
            return buffer
        shape = list(like.shape)
        shape[2] = (needed + cls.BLOCK - 1) // cls.BLOCK * cls.BLOCK
        grown = torch.zeros(shape, dtype=like.dtype, device=like.device)
        if buffer is not None:
            grown[:, :, : buffer.shape[2]] = buffer
        return grown

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        """Append [1, kv_heads, T, D] rows; the rows written so far."""
        needed = self.offset + keys.shape[2]
        self.keys = self._reserve(self.keys, needed, keys)
        self.values = self._reserve(self.values, needed, values)
        self.keys[:, :, self.offset : needed] = keys
        self.values[:, :, self.offset : needed] = values
        self.offset = needed
        return self.keys[:, :, :needed], self.values[:, :, :needed]

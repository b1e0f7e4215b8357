"""The rotary angle atlas, built where it is read and grown on demand.

Mirrors models/laguna/layers/attention.py:171-196,227-243 (`LagunaAttention.angles`,
`_angle_atlas`): one fp32 table of rows `[cos(theta) || sin(theta)]` per position, built
once, rebuilt when a position passes its last row, and read one row per step instead of
deriving the angles per layer. The arithmetic is the fp64 build of
tests/test_kernel_qk_norm_rope.py:51-66 (theta = pos * f_i in fp64, cos and sin rounded
once to fp32), the table the QK-norm + RoPE kernels are checked against:

- the frequencies f_i = exp(-ln(base) * i / P) (or 1 / freqs for a YaRN table, the
  reference's `freqs` argument) are computed once on the host in fp64;
- on a ROCm device the rows are filled by `omnia_rope_angle_atlas`; growing fills only
  the new rows, and keeps the old ones where they are (the table is reallocated at twice
  its rows or to the position asked for, whichever is more);
- on the CPU the same fp64 arithmetic runs in torch ops.

`table()` views the atlas as an `AngleTable` (the separate-table contract the HIP
strategies read in place); calling the atlas is the reference's `Angles` contract.
"""

from __future__ import annotations

import numpy as np
import torch

from ...runtime import ops
from .kernel import AngleTable

DEFAULT_ROWS = 4096  # models/laguna/layers/attention.py:226 (_ATLAS_ROWS)


def rope_frequencies(pairs: int, base: float) -> np.ndarray:
    """exp(-ln(base) * i / pairs) in fp64, i < pairs."""
    return np.exp(-np.log(base) * np.arange(pairs) / pairs)


class AngleAtlas:
    """A growable [rows, 2 * pairs] fp32 atlas on one device."""

    def __init__(self, pairs: int, *, base: float | None = None,
                 inverse_frequencies: np.ndarray | None = None, rows: int = DEFAULT_ROWS,
                 device: torch.device | str | None = None) -> None:
        if (base is None) == (inverse_frequencies is None):
            raise ValueError("AngleAtlas: give base or inverse_frequencies (YaRN freqs), not both")
        if base is not None:
            frequencies = rope_frequencies(pairs, base)
        else:
            frequencies = 1.0 / np.asarray(inverse_frequencies, dtype=np.float64)
        if frequencies.shape != (pairs,):
            raise ValueError(f"AngleAtlas: {frequencies.shape[0]} frequencies for {pairs} pairs")
        self.pairs = pairs
        self.device = torch.device(device if device is not None else "cpu")
        self.frequencies = torch.from_numpy(np.ascontiguousarray(frequencies)).to(self.device)
        self.atlas = torch.empty((0, 2 * pairs), dtype=torch.float32, device=self.device)
        self.grow(rows)

    @property
    def rows(self) -> int:
        return self.atlas.shape[0]

    def _fill(self, first: int, out: torch.Tensor) -> None:
        rows = out.shape[0]
        if rows == 0:
            return
        if self.device.type == "cuda":
            ops.rope_angle_atlas(self.frequencies, first, rows, out=out)
            return
        positions = torch.arange(first, first + rows, dtype=torch.float64)
        theta = positions[:, None] * self.frequencies[None, :].to(torch.float64)
        out[:, : self.pairs] = torch.cos(theta).to(torch.float32)
        out[:, self.pairs :] = torch.sin(theta).to(torch.float32)

    def grow(self, rows: int) -> None:
        """Make the atlas cover positions [0, rows), filling only the new rows."""
        old = self.rows
        if rows <= old:
            return
        if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f"AngleAtlas: cannot grow to {rows} rows under graph capture")
        atlas = torch.empty((rows, 2 * self.pairs), dtype=torch.float32, device=self.device)
        if old:
            atlas[:old].copy_(self.atlas)
        self._fill(old, atlas[old:])
        self.atlas = atlas

    def ensure(self, position: int) -> None:
        """Grow, if needed, so that row `position` exists (to twice the rows at least)."""
        if position >= self.rows:
            self.grow(max(2 * self.rows, position + 1))

    def table(self) -> AngleTable:
        return AngleTable.from_atlas(self.atlas)

    def __call__(self, offset: int, length: int) -> torch.Tensor:
        """Rows offset .. offset+length-1, cosines then sines (the `Angles` contract)."""
        self.ensure(offset + length - 1)
        return self.atlas[offset : offset + length]

"""The rotary angle atlas, built where it is read and grown on demand.

The reference's atlas (models/laguna/layers/attention.py:171-196,227-243,
`LagunaAttention.angles`, `_angle_atlas`) is one fp32 table of rows
`[cos(theta) || sin(theta)]` per position, built once, rebuilt when a position passes
its last row, and read one row per step instead of deriving the angles per layer. This
class keeps that contract (built once, grown past its last row, read by row) and offers
two arithmetics for the table's values:

- "fp64" (the default): theta = pos * f_i in fp64 and cos, sin rounded once to fp32, the
  table of tests/test_kernel_qk_norm_rope.py:51-66 that the reference checks its table
  rotation against, and the one the QK-norm + RoPE kernels here are tested with. The
  frequencies f_i = exp(-ln(base) * i / P) (or 1 / freqs for a YaRN table) are computed
  once on the host in fp64.
- "fp32": Laguna's own op order (attention.py:236-243): inverse_i = base ** (2i / D)
  and theta = fp32(pos) / inverse_i as fp32 operations (a YaRN `freqs` table is taken as
  the inverse row as given), then cos and sin of the fp32 angle; every operation
  correctly rounded. The fp32 quotient differs from the fp64 angle by up to half an fp32
  ulp of theta (up to about 2e-3 rad at position 32,768 and beyond), so the two tables
  differ visibly at long positions: max |cos diff| 3.2e-3 and max |sin diff| 3.2e-3 over
  40,960 rows x 64 pairs at base 1e6 (2.4e-4 below row 4,096). Neither is MLX's own
  bits (its cos and sin are Metal's), which no test here can pin.

On a ROCm device the rows are filled by `omnia_rope_angle_atlas` (fp64) or
`omnia_rope_angle_atlas_fp32`; growing fills only the new rows and keeps the old ones
where they are (the table is reallocated at twice its rows or to the position asked
for, whichever is more). On the CPU the same arithmetic runs in torch ops.

`table()` views the atlas as an `AngleTable` (the separate-table contract the HIP
strategies read in place); calling the atlas is the reference's `Angles` contract.
"""

from __future__ import annotations

from typing import Literal

import numpy as np
import torch

from ...runtime import ops
from .kernel import AngleTable

DEFAULT_ROWS = 4096  # models/laguna/layers/attention.py:226 (_ATLAS_ROWS)


def rope_frequencies(pairs: int, base: float) -> np.ndarray:
    """exp(-ln(base) * i / pairs) in fp64, i < pairs."""
    return np.exp(-np.log(base) * np.arange(pairs) / pairs)


def rope_inverse_fp32(pairs: int, base: float) -> np.ndarray:
    """Laguna's `base ** (arange(0, D, 2) / D)` as fp32 operations, each correctly rounded:
    the exponent 2i / D as an fp32 quotient, then the fp32 power (evaluated in fp64 from
    the fp32 base and exponent, rounded once)."""
    exponents = (np.arange(0, 2 * pairs, 2, dtype=np.float32) / np.float32(2 * pairs)).astype(np.float32)
    return np.power(np.float64(np.float32(base)), exponents.astype(np.float64)).astype(np.float32)


class AngleAtlas:
    """A growable [rows, 2 * pairs] fp32 atlas on one device."""

    def __init__(self, pairs: int, *, base: float | None = None,
                 inverse_frequencies: np.ndarray | None = None, rows: int = DEFAULT_ROWS,
                 device: torch.device | str | None = None,
                 arithmetic: Literal["fp64", "fp32"] = "fp64") -> None:
        if (base is None) == (inverse_frequencies is None):
            raise ValueError("AngleAtlas: give base or inverse_frequencies (YaRN freqs), not both")
        if arithmetic not in ("fp64", "fp32"):
            raise ValueError(f"AngleAtlas: arithmetic must be 'fp64' or 'fp32', not {arithmetic!r}")
        if arithmetic == "fp64":
            frequencies = (rope_frequencies(pairs, base) if base is not None
                           else 1.0 / np.asarray(inverse_frequencies, dtype=np.float64))
        else:
            frequencies = (rope_inverse_fp32(pairs, base) if base is not None
                           else np.asarray(inverse_frequencies, dtype=np.float32))
        if frequencies.shape != (pairs,):
            raise ValueError(f"AngleAtlas: {frequencies.shape[0]} frequencies for {pairs} pairs")
        self.pairs = pairs
        self.arithmetic = arithmetic
        self.device = torch.device(device if device is not None else "cpu")
        # fp64: the frequencies f_i; fp32: the inverse row base ** (2i / D).
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
            if self.arithmetic == "fp64":
                ops.rope_angle_atlas(self.frequencies, first, rows, out=out)
            else:
                ops.rope_angle_atlas_fp32(self.frequencies, first, rows, out=out)
            return
        positions = torch.arange(first, first + rows, dtype=torch.float64)
        if self.arithmetic == "fp64":
            theta = positions[:, None] * self.frequencies[None, :].to(torch.float64)
        else:
            theta = (positions.to(torch.float32).to(torch.float64)[:, None]
                     / self.frequencies[None, :].to(torch.float64)).to(torch.float32).to(torch.float64)
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

"""Writes the small golden fixtures under tests/golden/ from the CPU oracle.

The reference (mlx-omnia) holds no golden tensors for these kernels and cannot run here
(no MLX, Python 3.10, Metal-only kernels), so the vectors are produced by this repo's
own oracle on seeded inputs and serve as regression pins: `tests/test_golden.py`
recomputes them on the CPU and the GPU tests compare the HIP kernels with them.
Run: `python tests/golden/make_golden.py`.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import add_norm  # noqa: E402
from oracle.bf16 import from_float  # noqa: E402


def make_add_norm() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(1)
    rows, hidden, eps = 4, 2560, 1e-6
    x = from_float(rng.standard_normal((rows, hidden)))
    branch = from_float(rng.standard_normal((rows, hidden)))
    weight = from_float(1.0 + 0.1 * rng.standard_normal(hidden))
    summed, normalized = add_norm.add_rms_norm(x, branch, weight, eps)
    return dict(x=x, branch=branch, weight=weight, eps=np.float32(eps),
                summed=summed, normalized=normalized)


MAKERS = {"add_norm": make_add_norm}


def main(names: list[str]) -> None:
    for name in names or list(MAKERS):
        arrays = MAKERS[name]()
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
        print(f"wrote tests/golden/{name}.npz", flush=True)


if __name__ == "__main__":
    main(sys.argv[1:])

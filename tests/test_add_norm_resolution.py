"""Facade resolution and the Core chain of the residual join, on the CPU.

Mirrors tests/test_kernel_add_rms_norm.py:59-91 (predicates and resolution by
declaration): a CPU declaration resolves to the Core chain, `reference=True` forces it,
and the HIP predicate accepts exactly the hidden sizes the kernel tiles.
"""

import numpy as np
import pytest
import torch

from mlx_omnia_amd.kernels import RESOLVED
from mlx_omnia_amd.kernels.add_norm import AddRmsNorm, DefaultAddRmsNorm, applies
from mlx_omnia_amd.kernels.leaf import RMSNormLeaf
from oracle import add_norm as oracle
from oracle.bf16 import from_float, ulp_distance


def test_predicate():
    for hidden in (8, 1024, 2048, 2560, 2880, 4096, 8192):
        assert applies(hidden)
    for hidden in (0, 4, 100, 8200, 16384):
        assert not applies(hidden)


def test_cpu_declaration_resolves_to_core_chain():
    leaf = RMSNormLeaf(torch.ones(2560, dtype=torch.bfloat16), 1e-6)
    assert isinstance(AddRmsNorm(leaf).strategy, DefaultAddRmsNorm)
    assert isinstance(AddRmsNorm(leaf, tokens=1, reference=True).strategy, DefaultAddRmsNorm)
    assert "mlx_omnia_amd.kernels.add_norm.default" in RESOLVED


@pytest.mark.parametrize("rows,hidden", [(1, 2560), (9, 2048)])
def test_core_chain_matches_oracle(rows, hidden):
    rng = np.random.default_rng(rows)
    x, b = from_float(rng.standard_normal((rows, hidden))), from_float(rng.standard_normal((rows, hidden)))
    w = from_float(1 + 0.1 * rng.standard_normal(hidden))
    t = lambda bits: torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    join = AddRmsNorm(RMSNormLeaf(t(w), 1e-6))
    s, n = join(t(x), t(b))
    want_s, want_n = oracle.add_rms_norm(x, b, w, 1e-6)
    bits = lambda v: v.view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bits(s), want_s)
    assert ulp_distance(bits(n), want_n).max() <= 1

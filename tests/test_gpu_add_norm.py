"""HIP residual add + RMSNorm against the CPU oracle (through the facade and the C ABI).

The bar: the residual sum is bit-exact; the normalised output is within 2 bf16 ulp and
atol/rtol 1e-2 of the oracle (the only free difference is the fp32 summation order of
the sum of squares). Shapes cover the configs (T=1 decode, T=512 prefill at H=2560),
other checkpoint widths, a hidden size whose last 16-byte vectors fill only part of the
wave (2880), the smallest row (8) and the largest the kernel serves (8192), and empty input.
"""

import numpy as np
import pytest
import torch

from mlx_omnia_amd.kernels.add_norm import AddRmsNorm, HipAddRmsNorm
from mlx_omnia_amd.kernels.leaf import RMSNormLeaf
from mlx_omnia_amd.runtime import ops
from oracle import add_norm as oracle
from oracle.bf16 import from_float, to_f32
from util import assert_bf16_close, bits_of, exact_fraction, to_device

pytestmark = pytest.mark.gpu

EPS = 1e-6
SHAPES = [(1, 2560), (512, 2560), (7, 2048), (3, 4096), (5, 8), (2, 8192), (33, 2880), (4100, 2560)]


def _inputs(rows, hidden, seed):
    rng = np.random.default_rng(seed)
    return (
        from_float(rng.standard_normal((rows, hidden))),
        from_float(rng.standard_normal((rows, hidden))),
        from_float(1.0 + 0.1 * rng.standard_normal(hidden)),
    )


@pytest.mark.parametrize("rows,hidden", SHAPES)
def test_matches_oracle(rows, hidden):
    print(f"add_rms_norm rows={rows} hidden={hidden}", flush=True)
    x, b, w = _inputs(rows, hidden, seed=rows * 7 + hidden)
    join = AddRmsNorm(RMSNormLeaf(to_device(w), EPS), tokens=1 if rows == 1 else None)
    assert isinstance(join.strategy, HipAddRmsNorm)
    s, n = join(to_device(x), to_device(b))
    torch.cuda.synchronize()
    want_s, want_n = oracle.add_rms_norm(x, b, w, EPS)
    assert np.array_equal(bits_of(s), want_s)
    assert_bf16_close(bits_of(n), want_n)
    assert exact_fraction(bits_of(n), want_n) > 0.99


def test_checkpoint_magnitudes_and_keeps_shape():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((1, 3, 2048)) * 30.0
    x += rng.standard_normal(x.shape) * 300.0 * (rng.uniform(size=x.shape) > 0.99)
    xb, bb = from_float(x), from_float(rng.standard_normal(x.shape) * 3.0)
    w = from_float(1.0 + 0.2 * rng.standard_normal(2048))
    s, n = AddRmsNorm(RMSNormLeaf(to_device(w), EPS))(to_device(xb), to_device(bb))
    assert s.shape == (1, 3, 2048) and n.shape == (1, 3, 2048)
    want_s, want_n = oracle.add_rms_norm(xb.reshape(-1, 2048), bb.reshape(-1, 2048), w, EPS)
    assert np.array_equal(bits_of(s).reshape(-1, 2048), want_s)
    assert_bf16_close(bits_of(n).reshape(-1, 2048), want_n)


def test_eps_reaches_the_kernel():
    x, b, w = _inputs(2, 2048, seed=4)
    x, b = from_float(to_f32(x) * 1e-3), from_float(to_f32(b) * 1e-3)
    s, n = AddRmsNorm(RMSNormLeaf(to_device(w), 0.5))(to_device(x), to_device(b))
    _, want = oracle.add_rms_norm(x, b, w, 0.5)
    _, without = oracle.add_rms_norm(x, b, w, EPS)
    assert_bf16_close(bits_of(n), want)
    assert not np.array_equal(bits_of(n), without)


def test_empty_rows_and_rejections():
    w = to_device(from_float(np.ones(2560)))
    empty = torch.empty((0, 2560), dtype=torch.bfloat16, device="cuda")
    s, n = ops.add_rms_norm(empty, empty, w, EPS)
    assert s.shape == (0, 2560) and n.shape == (0, 2560)
    bad = torch.zeros((2, 100), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        ops.add_rms_norm(bad, bad, torch.ones(100, dtype=torch.bfloat16, device="cuda"), EPS)


def test_golden_fixture():
    golden = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "add_norm.npz")
    s, n = ops.add_rms_norm(
        to_device(golden["x"]), to_device(golden["branch"]), to_device(golden["weight"]),
        float(golden["eps"]),
    )
    assert np.array_equal(bits_of(s), golden["summed"])
    assert_bf16_close(bits_of(n), golden["normalized"])

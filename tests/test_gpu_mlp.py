"""HIP dense SwiGLU MLP (csrc/mlp.hip) against the oracle (oracle/mlp.py).

gate_up_swiglu sums in fp32 in its own order where the oracle rounds the exact dot
product once; the two agree except where a projection sits at a bf16 rounding boundary,
and the bf16 SwiGLU chain then carries that ulp on. down_residual adds one more fp32
sum. Both use the north-star bf16 bar (assert_bf16_close) with at least 99% of the
outputs bit-identical.

Shapes: Qwen3-4B's MLP (hidden 2560, inner 9728, the bench workload), Qwen3-0.6B's
(1024, 3072), the reference test's (256, 512), ragged sizes that leave lanes idle and
an odd pair count, hidden 8192 (one pair per wave), and a down projection with
inner 25600 (seven chunks of the contraction).
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from mlx_omnia_amd.kernels.leaf import SwiGLU
from mlx_omnia_amd.kernels.mlp import HipDenseMlp, Mlp
from mlx_omnia_amd.runtime import ops
from oracle import mlp
from oracle.bf16 import from_float
from util import assert_bf16_close, bits_of, to_device

pytestmark = pytest.mark.gpu


def _weight(rows, cols, seed, scale):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    values = torch.randn((rows, cols), generator=gen, device="cuda", dtype=torch.float32)
    return (scale * values).to(torch.bfloat16)


GATE_UP_SHAPES = [
    # hidden, inner, seed
    (2560, 9728, 1),
    (1024, 3072, 2),
    (256, 512, 3),
    (520, 75, 4),     # 65 vectors per row, an odd pair count
    (8192, 64, 5),    # 16 vectors per lane: one pair per wave
    (8, 1, 6),
]


@pytest.mark.parametrize("hidden,inner,seed", GATE_UP_SHAPES)
def test_gate_up_swiglu_matches_oracle(hidden, inner, seed):
    print(f"dense_gate_up_swiglu H={hidden} I={inner}", flush=True)
    rng = np.random.default_rng(seed)
    fused = _weight(2 * inner, hidden, seed, 1.5 / np.sqrt(hidden))
    x = from_float(rng.standard_normal(hidden))
    got = bits_of(ops.dense_gate_up_swiglu(to_device(x), fused))
    want = mlp.gate_up_swiglu(x, bits_of(fused))
    assert got.shape == (inner,)
    assert_bf16_close(got, want, min_exact=0.99)


DOWN_SHAPES = [
    (2560, 9728, 11),
    (1024, 3072, 12),
    (256, 512, 13),
    (77, 72, 14),     # odd row count, 9 vectors per row
    (1024, 25600, 15),
    (3, 8, 16),
]


@pytest.mark.parametrize("hidden,inner,seed", DOWN_SHAPES)
def test_down_residual_matches_oracle(hidden, inner, seed):
    print(f"dense_down_residual H={hidden} I={inner}", flush=True)
    rng = np.random.default_rng(seed)
    down = _weight(hidden, inner, seed, 1.0 / np.sqrt(inner))
    act = from_float(rng.standard_normal(inner))
    residual = from_float(rng.standard_normal(hidden))
    got = bits_of(ops.dense_down_residual(to_device(act), down, to_device(residual)))
    want = mlp.down_residual(act, bits_of(down), residual)
    assert got.shape == (hidden,)
    assert_bf16_close(got, want, min_exact=0.99)


def test_zero_activation_returns_the_residual_and_layout_is_gate_first():
    hidden, inner = 512, 256
    rng = np.random.default_rng(21)
    down = _weight(hidden, inner, 21, 0.1)
    residual = from_float(rng.standard_normal(hidden))
    zeros = torch.zeros(inner, dtype=torch.bfloat16, device="cuda")
    out = bits_of(ops.dense_down_residual(zeros, down, to_device(residual)))
    assert np.array_equal(out, residual)
    # SwiGLU is asymmetric in gate and up: swapping the halves of the stack must change it.
    fused = _weight(2 * inner, hidden, 22, 0.05)
    x = to_device(from_float(rng.standard_normal(hidden)))
    a = bits_of(ops.dense_gate_up_swiglu(x, fused))
    b = bits_of(ops.dense_gate_up_swiglu(x, torch.cat([fused[inner:], fused[:inner]]).contiguous()))
    assert (a != b).mean() > 0.9


def test_facade_resolves_to_hip_and_matches_oracle():
    hidden, inner = 2560, 9728
    rng = np.random.default_rng(23)
    leaf = SwiGLU(hidden, inner).to(device="cuda", dtype=torch.bfloat16)
    mlp_facade = Mlp(leaf, hidden=hidden, inner=inner)
    assert isinstance(mlp_facade.strategy, HipDenseMlp)
    assert not isinstance(Mlp(leaf, hidden=hidden, inner=inner, activation="gelu_tanh").strategy,
                          HipDenseMlp)
    x = from_float(rng.standard_normal(hidden))
    residual = from_float(rng.standard_normal(hidden))
    with torch.no_grad():
        out = bits_of(mlp_facade(to_device(x), to_device(residual)))
    fused = bits_of(leaf.gate_up_proj.weight)
    down = bits_of(leaf.down_proj.weight)
    act = bits_of(ops.dense_gate_up_swiglu(to_device(x), leaf.gate_up_proj.weight.detach()))
    assert_bf16_close(act, mlp.gate_up_swiglu(x, fused), min_exact=0.99)
    assert_bf16_close(out, mlp.down_residual(act, down, residual), min_exact=0.99)


def test_golden_fixture():
    golden = np.load(Path(__file__).parent / "golden" / "mlp.npz")
    act = bits_of(ops.dense_gate_up_swiglu(to_device(golden["x"]), to_device(golden["fused_weight"])))
    assert_bf16_close(act, golden["act"], min_exact=0.99)
    out = bits_of(ops.dense_down_residual(to_device(golden["act"]), to_device(golden["down_weight"]),
                                          to_device(golden["residual"])))
    assert_bf16_close(out, golden["out"], min_exact=0.99)

"""HIP SwiGLU and gate-softplus against the oracle, bit-exact.

Both kernels evaluate every rounding step correctly rounded (the sigmoid to bf16, each
fp32 step of the softplus chain), so the outputs are compared bit for bit. Cases: the
configs (gate/up [8192, 9728] ~N(0,1); a [8192, 32] ~N(0,1), A_log ~U(0, 2.7), dt_bias
~N(0, 0.5)), the halves of a fused projection, special values, a head count that is not
a multiple of 8, empty input, and the facades' resolution.
"""

import numpy as np
import pytest
import torch

from mlx_omnia_amd.kernels.gate_softplus import GateSoftplus, HipGateSoftplus
from mlx_omnia_amd.kernels.gate_up import GateUpActivation, HipSwiGLU
from mlx_omnia_amd.runtime import ops
from oracle import activations as act
from oracle.bf16 import from_float, to_f32
from util import bits_of, f32_to_device, to_device

pytestmark = pytest.mark.gpu


def test_swiglu_config_bit_exact():
    print("swiglu config [8192, 9728]", flush=True)
    rng = np.random.default_rng(5)
    g = from_float(rng.standard_normal((8192, 9728), dtype=np.float32))
    u = from_float(rng.standard_normal((8192, 9728), dtype=np.float32))
    y = ops.swiglu(to_device(g), to_device(u))
    torch.cuda.synchronize()
    got = bits_of(y)
    del y
    want = act.swiglu(g, u)
    assert np.array_equal(got, want), f"{int((got != want).sum())} elements differ"


def test_swiglu_fused_halves_and_specials_via_facade():
    rng = np.random.default_rng(6)
    fused = rng.standard_normal((33, 2 * 520)).astype(np.float32) * 6
    fused[0, :8] = [0.0, -0.0, 88.0, -88.0, 90.0, -90.0, 1e-30, -1e-30]
    fused[1, :3] = [np.inf, -np.inf, np.nan]
    # inf gates against zero, negative, positive and infinite ups; a NaN up.
    fused[2, :6] = [np.inf, np.inf, -np.inf, -np.inf, 100.0, 3.0]
    fused[2, 520:526] = [0.0, -3.0, 2.0, np.inf, np.inf, np.nan]
    bits = from_float(fused)
    activation = GateUpActivation()
    assert isinstance(activation.strategy, HipSwiGLU)
    y = activation(to_device(bits))
    want = act.swiglu(bits[:, :520], bits[:, 520:])

    def same(got):
        # NaN exactly where the oracle has NaN (its sign and payload are the platform's:
        # x86 makes -inf * 0 a negative NaN, the GPU a positive one); every other element,
        # infinities included, bit for bit.
        nan = np.isnan(to_f32(want))
        assert np.array_equal(np.isnan(to_f32(got)), nan)
        assert np.array_equal(got[~nan], want[~nan])
        assert nan.any() and np.isinf(to_f32(want)).any()

    same(bits_of(y))
    # Separate tensors with row strides, one row, empty.
    y2 = ops.swiglu(to_device(bits)[:, :520], to_device(bits)[:, 520:])
    same(bits_of(y2))
    assert ops.swiglu(to_device(bits[:0, :8]), to_device(bits[:0, :8])).shape == (0, 8)


def test_gate_softplus_config_bit_exact():
    rng = np.random.default_rng(7)
    a = from_float(rng.standard_normal((8192, 32)))
    a_log = rng.uniform(0, 2.7, 32).astype(np.float32)
    dt_bias = (0.5 * rng.standard_normal(32)).astype(np.float32)
    gate = GateSoftplus(f32_to_device(a_log), f32_to_device(dt_bias))
    assert isinstance(gate.strategy, HipGateSoftplus)
    g = gate(to_device(a))
    assert g.dtype == torch.float32 and g.shape == (8192, 32)
    assert np.array_equal(g.cpu().numpy(), act.gate_softplus(a, a_log, dt_bias))


def test_gate_softplus_scalar_path_and_specials():
    rng = np.random.default_rng(8)
    values = rng.standard_normal((7, 12)).astype(np.float32) * 30
    values[0, :6] = [np.inf, -np.inf, np.nan, 0.0, -0.0, 1e-30]
    a = from_float(values)
    a_log = rng.uniform(0, 2.7, 12).astype(np.float32)
    dt_bias = (0.5 * rng.standard_normal(12)).astype(np.float32)
    got = ops.gate_softplus(to_device(a), f32_to_device(a_log), f32_to_device(dt_bias)).cpu().numpy()
    want = act.gate_softplus(a, a_log, dt_bias)
    assert np.array_equal(got, want, equal_nan=True)
    empty = ops.gate_softplus(to_device(a[:0]), f32_to_device(a_log), f32_to_device(dt_bias))
    assert empty.shape == (0, 12)


@pytest.mark.parametrize("rows,heads,pad", [(130, 6, 0), (3, 258, 2), (5, 600, 4), (257, 32, 6)])
def test_gate_softplus_grid_shapes(rows, heads, pad):
    """Pair counts that fill part of a workgroup's columns (the rest of it rows), span two
    column blocks, or pass the decay table's 256 heads; rows that end mid-block; a row
    stride past the heads. The fused launch's gate-softplus part on the same inputs."""
    print(f"gate_softplus rows={rows} heads={heads} pad={pad}", flush=True)
    rng = np.random.default_rng(heads + rows)
    values = rng.standard_normal((rows, heads + pad)).astype(np.float32) * 8
    a = from_float(values)
    a_log = rng.uniform(0, 2.7, heads).astype(np.float32)
    dt_bias = (0.5 * rng.standard_normal(heads)).astype(np.float32)
    want = act.gate_softplus(a[:, :heads], a_log, dt_bias)
    dev = to_device(a)[:, :heads]
    got = ops.gate_softplus(dev, f32_to_device(a_log), f32_to_device(dt_bias)).cpu().numpy()
    assert np.array_equal(got, want)
    up = to_device(from_float(rng.standard_normal((2, 16)).astype(np.float32)))
    _, g = ops.gated_activations(up, up, dev, f32_to_device(a_log), f32_to_device(dt_bias))
    assert np.array_equal(g.cpu().numpy(), want)


def test_golden_fixture():
    golden = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "activations.npz")
    y = ops.swiglu(to_device(golden["gate"]), to_device(golden["up"]))
    assert np.array_equal(bits_of(y), golden["swiglu"])
    g = ops.gate_softplus(to_device(golden["a"]), f32_to_device(golden["a_log"]),
                          f32_to_device(golden["dt_bias"]))
    assert np.array_equal(g.cpu().numpy(), golden["gate_softplus"])

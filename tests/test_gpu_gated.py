"""Both gated activations in one dispatch, against the oracle and the single kernels.

`omnia_gated_activations` computes exactly what `omnia_swiglu` and `omnia_gate_softplus`
compute, so its two outputs are compared bit for bit with the oracle:
- at configs[3] (gate/up [8192, 9728] and a [8192, 32]);
- on the halves of a fused projection with special values;
- with either part empty.
The facade binds the fused launch only where both single bindings bind. A call the
fused kernel does not take (an odd head count) runs the two single kernels and is
recorded.
"""

import importlib

import numpy as np
import pytest
import torch

from mlx_omnia_amd.kernels.gated import (DefaultGatedActivations, GatedActivations,
                                         HipGatedActivations)
from mlx_omnia_amd.runtime import ops
from oracle import activations as act
from oracle.bf16 import from_float, to_f32
from util import bits_of, f32_to_device, to_device

pytestmark = pytest.mark.gpu


def _gate_params(rng, heads):
    return (rng.uniform(0, 2.7, heads).astype(np.float32),
            (0.5 * rng.standard_normal(heads)).astype(np.float32))


def test_config_pair_bit_exact_in_one_launch():
    print("gated_activations config [8192, 9728] + [8192, 32]", flush=True)
    rng = np.random.default_rng(5)
    g = from_float(rng.standard_normal((8192, 9728), dtype=np.float32))
    u = from_float(rng.standard_normal((8192, 9728), dtype=np.float32))
    a = from_float(rng.standard_normal((8192, 32)))
    a_log, dt_bias = _gate_params(rng, 32)
    pair = GatedActivations(f32_to_device(a_log), f32_to_device(dt_bias))
    assert isinstance(pair.strategy, HipGatedActivations)
    y, gate = pair(to_device(g), to_device(u), to_device(a))
    torch.cuda.synchronize()
    got_y, got_g = bits_of(y), gate.cpu().numpy()
    del y, gate
    assert np.array_equal(got_g, act.gate_softplus(a, a_log, dt_bias))
    want = act.swiglu(g, u)
    assert np.array_equal(got_y, want), f"{int((got_y != want).sum())} elements differ"


def test_fused_halves_specials_and_empty_parts():
    rng = np.random.default_rng(6)
    fused = rng.standard_normal((33, 2 * 520)).astype(np.float32) * 6
    fused[0, :8] = [0.0, -0.0, 88.0, -88.0, 90.0, -90.0, 1e-30, -1e-30]
    fused[1, :3] = [np.inf, -np.inf, np.nan]
    bits = from_float(fused)
    values = rng.standard_normal((19, 12)).astype(np.float32) * 30
    values[0, :6] = [np.inf, -np.inf, np.nan, 0.0, -0.0, 1e-30]
    a = from_float(values)
    a_log, dt_bias = _gate_params(rng, 12)
    dev = to_device(bits)
    y, gate = ops.gated_activations(dev[:, :520], dev[:, 520:], to_device(a),
                                    f32_to_device(a_log), f32_to_device(dt_bias))
    want = act.swiglu(bits[:, :520], bits[:, 520:])
    got = bits_of(y)
    nan = np.isnan(to_f32(want))  # NaN's sign and payload are the platform's
    assert np.array_equal(np.isnan(to_f32(got)), nan)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.array_equal(gate.cpu().numpy(), act.gate_softplus(a, a_log, dt_bias), equal_nan=True)
    # Each part alone: the other part empty.
    y0, g0 = ops.gated_activations(dev[:0, :520], dev[:0, 520:], to_device(a),
                                   f32_to_device(a_log), f32_to_device(dt_bias))
    assert y0.shape == (0, 520)
    assert np.array_equal(g0.cpu().numpy(), act.gate_softplus(a, a_log, dt_bias), equal_nan=True)
    y1, g1 = ops.gated_activations(dev[:, :520], dev[:, 520:], to_device(a[:0]),
                                   f32_to_device(a_log), f32_to_device(dt_bias))
    assert g1.shape == (0, 12)
    assert np.array_equal(np.isnan(to_f32(bits_of(y1))), nan)


def test_odd_heads_run_the_single_kernels_and_are_recorded():
    rng = np.random.default_rng(9)
    g = from_float(rng.standard_normal((5, 64), dtype=np.float32))
    u = from_float(rng.standard_normal((5, 64), dtype=np.float32))
    a = from_float(rng.standard_normal((5, 7)))
    a_log, dt_bias = _gate_params(rng, 7)
    pair = GatedActivations(f32_to_device(a_log), f32_to_device(dt_bias))
    assert isinstance(pair.strategy, HipGatedActivations)
    resolve = importlib.import_module("mlx_omnia_amd.kernels.resolve")
    before = sum(resolve.FALLBACKS.values())
    y, gate = pair(to_device(g), to_device(u), to_device(a))
    assert sum(resolve.FALLBACKS.values()) == before + 1
    assert np.array_equal(bits_of(y), act.swiglu(g, u))
    assert np.array_equal(gate.cpu().numpy(), act.gate_softplus(a, a_log, dt_bias))
    # A clamped SwiGLU is other arithmetic: the pair declines to the Core chains.
    clamped = GatedActivations(f32_to_device(a_log), f32_to_device(dt_bias), limit=7.0)
    assert isinstance(clamped.strategy, DefaultGatedActivations)

"""The dense MLP oracle (oracle/mlp.py) pinned without its own formula.

- The bf16 SwiGLU chain: values derived by hand from its definition (g = 1, 2, -1 with
  u = 1), torch's bf16 tensor ops (each op computes in float and rounds to bf16, as the
  reference's `bfloat` temporaries do), the special values (signed zeros, exp overflow).
- The projections: torch's float64 matmul, rounded once; a one-hot row picks a weight.
- The reference's own layout test (tests/test_kernel_dense_mlp.py:87-101): gate rows
  first, so the swapped chain must disagree; and its op-chain comparison at its shapes
  (HIDDEN 256, INNER 512) under its floor, relative_diff < 2^-7.
- Planted mistakes (an fp32 SwiGLU, a dropped residual, gate and up swapped) fail.
"""

import numpy as np
import pytest
import torch

from oracle import mlp
from oracle.bf16 import from_float, to_f32, ulp_distance
from util import relative_diff

HIDDEN, INNER = 256, 512


def _torch_bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_swiglu_steps_hand_values():
    # g = 1: exp(1) -> 2.71875, 1 + e = 3.71875, 1/3.71875 -> 0.26953125, 1 - y = 0.73046875.
    # g = 2: exp(2) -> 7.375, 8.375, 1/8.375 -> 0.11962890625, 1 - y -> 0.87890625, x2.
    # g = -1: the negative branch keeps y: -1 * 0.26953125.
    got = to_f32(mlp.swiglu_steps(from_float([1.0, 2.0, -1.0]), from_float([1.0, 1.0, 1.0])))
    assert got.tolist() == [0.73046875, 1.7578125, -0.26953125]


def test_swiglu_steps_special_values():
    g = from_float([0.0, -0.0, 100.0, -100.0, 89.0])
    u = from_float([3.0, 3.0, 1.5, 2.0, 1.0])
    got = to_f32(mlp.swiglu_steps(g, u))
    assert got[0] == 0.0 and not np.signbit(got[0])
    assert got[1] == 0.0 and np.signbit(got[1])          # -0 * 0.5 * 3
    assert got[2] == np.float32(150.0)                   # exp overflows: sigmoid 1
    assert got[3] == 0.0 and np.signbit(got[3])          # y = 0: silu = -0
    assert got[4] == np.float32(89.0)


def test_swiglu_steps_match_torch_bf16_ops():
    rng = np.random.default_rng(0)
    g = from_float(3 * rng.standard_normal(20000))
    u = from_float(rng.standard_normal(20000))
    tg, tu = _torch_bf16(g), _torch_bf16(u)
    e = torch.exp(tg.abs())
    den = 1.0 + e
    y = 1.0 / den
    sig = torch.where(tg < 0, y, 1.0 - y)
    want = _bits((tg * sig) * tu)
    got = mlp.swiglu_steps(g, u)
    assert ((tg * sig).dtype, want.dtype) == (torch.bfloat16, np.uint16)
    # torch's float exp can land on the other side of a bf16 tie than the exact value.
    assert ulp_distance(got, want).max() <= 1
    assert (got == want).mean() > 0.999


def test_projections_match_torch_float64():
    rng = np.random.default_rng(1)
    x = from_float(rng.standard_normal(HIDDEN))
    w = from_float(0.1 * rng.standard_normal((2 * INNER, HIDDEN)))
    want = (torch.from_numpy(to_f32(w)).double() @ torch.from_numpy(to_f32(x)).double()).float()
    got = mlp.project(x, w)
    assert ulp_distance(got, from_float(want.numpy())).max() <= 1
    one_hot = np.zeros(HIDDEN, dtype=np.uint16)
    one_hot[5] = from_float([1.0])[0]
    assert np.array_equal(mlp.project(one_hot, w), w[:, 5])


def test_reference_op_chain_floor_and_layout():
    """tests/test_kernel_dense_mlp.py:64-101 restated on torch: fp32 projections, then the
    bf16-step chain; the swapped reference must exceed the floor."""
    rng = np.random.default_rng(2)
    gate = from_float(0.1 * rng.standard_normal((INNER, HIDDEN)))
    up = from_float(0.1 * rng.standard_normal((INNER, HIDDEN)))
    x = from_float(rng.standard_normal(HIDDEN))
    got = to_f32(mlp.gate_up_swiglu(x, np.concatenate([gate, up])))
    xf = torch.from_numpy(to_f32(x))
    g = (torch.from_numpy(to_f32(gate)) @ xf).to(torch.bfloat16)
    u = (torch.from_numpy(to_f32(up)) @ xf).to(torch.bfloat16)

    def chain(a, b):
        y = 1.0 / (1.0 + torch.exp(a.abs()))
        return ((a * torch.where(a < 0, y, 1.0 - y)) * b).float().numpy()

    assert relative_diff(got, chain(g, u)) < 2.0**-7
    assert relative_diff(got, chain(u, g)) > 2.0**-7


def test_down_residual_matches_torch_and_invariants():
    rng = np.random.default_rng(3)
    act = from_float(rng.standard_normal(INNER))
    w = from_float(0.1 * rng.standard_normal((HIDDEN, INNER)))
    residual = from_float(rng.standard_normal(HIDDEN))
    got = mlp.down_residual(act, w, residual)
    d = (torch.from_numpy(to_f32(w)).double() @ torch.from_numpy(to_f32(act)).double())
    want = (d.to(torch.bfloat16) + _torch_bf16(residual)).to(torch.bfloat16)
    assert ulp_distance(got, _bits(want)).max() <= 1
    assert (got == _bits(want)).mean() > 0.99
    zeros = np.zeros(INNER, dtype=np.uint16)
    assert np.array_equal(mlp.down_residual(zeros, w, residual), residual)
    eye = from_float(np.eye(HIDDEN, INNER))  # row n picks act[n]
    assert np.array_equal(mlp.down_residual(act, eye, np.zeros(HIDDEN, np.uint16)), act[:HIDDEN])


@pytest.mark.parametrize("kind", ["fp32_swiglu", "no_residual", "swapped"])
def test_planted_mistakes_fail(kind):
    rng = np.random.default_rng(4)
    x = from_float(rng.standard_normal(HIDDEN))
    fused = from_float(0.1 * rng.standard_normal((2 * INNER, HIDDEN)))
    down = from_float(0.05 * rng.standard_normal((HIDDEN, INNER)))
    residual = from_float(rng.standard_normal(HIDDEN))
    good = mlp.gate_up_swiglu(x, fused)
    if kind == "fp32_swiglu":
        p = to_f32(mlp.project(x, fused))
        g, u = p[:INNER], p[INNER:]
        bad = from_float(g / (1 + np.exp(-g)) * u)
        assert (bad != good).mean() > 0.05
    elif kind == "no_residual":
        out = mlp.down_residual(good, down, residual)
        assert not np.array_equal(out, mlp.down_residual(good, down, np.zeros_like(residual)))
    else:
        swapped = np.concatenate([fused[INNER:], fused[:INNER]])
        assert not np.array_equal(good, mlp.gate_up_swiglu(x, swapped))

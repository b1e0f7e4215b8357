"""The routed-expert oracle (oracle/moe.py) pinned without its own formula.

- gate_up: torch's float64 matmul of the gathered expert matrices, rounded once (the
  same exact dot product by another route); a one-hot row picks a weight column exactly;
  an invalid expert id gives a zero row.
- down_combine: torch's float32 restatement of the Metal expression and float64 matmul;
  zero routing weights return the residual; an identity down matrix returns the
  activation itself (scaled and rounded); the expert order of the sum; planted
  mistakes (gate/up swapped, the routing weight dropped, the residual dropped) fail.
"""

import numpy as np
import pytest
import torch

from oracle import moe
from oracle.bf16 import from_float, to_f32, ulp_distance

HIDDEN, INNER, EXPERTS, K = 64, 24, 6, 3


def _weights(rng, experts, out, inp, scale=0.05):
    return from_float(scale * rng.standard_normal((experts, out, inp)))


def test_gate_up_matches_torch_float64():
    rng = np.random.default_rng(0)
    x = from_float(rng.standard_normal(HIDDEN))
    w = _weights(rng, EXPERTS, 2 * INNER, HIDDEN)
    chosen = np.array([4, 0, 5], dtype=np.int32)
    got = moe.gate_up(x, w, chosen)
    rows = torch.from_numpy(to_f32(w)).double()[torch.from_numpy(chosen).long()]
    want = (rows @ torch.from_numpy(to_f32(x)).double()).float()
    assert got.shape == (K, 2 * INNER)
    # float64 -> bf16 in one rounding vs float64 -> fp32 -> bf16: equal unless a value sits
    # within an fp32 ulp of a bf16 midpoint.
    assert ulp_distance(got, from_float(want.numpy())).max() <= 1
    assert (got == from_float(want.numpy())).mean() > 0.99


def test_gate_up_one_hot_row_and_invalid_expert():
    rng = np.random.default_rng(1)
    w = _weights(rng, EXPERTS, 2 * INNER, HIDDEN)
    x = np.zeros(HIDDEN, dtype=np.uint16)
    x[17] = from_float(np.array([1.0]))[0]
    got = moe.gate_up(x, w, np.array([2, 7, -1], dtype=np.int32))
    assert np.array_equal(got[0], w[2, :, 17])
    assert np.all(to_f32(got[1:]) == 0.0)


def _down_inputs(rng, k=K):
    act = from_float(2 * rng.standard_normal((k, 2 * INNER)))
    w = _weights(rng, EXPERTS, HIDDEN, INNER)
    chosen = rng.choice(EXPERTS, size=k, replace=False).astype(np.int32)
    weights = rng.dirichlet(np.ones(k)).astype(np.float32)
    residual = from_float(rng.standard_normal(HIDDEN))
    return act, w, chosen, weights, residual


def test_down_combine_matches_torch_restatement():
    rng = np.random.default_rng(2)
    act, w, chosen, weights, residual = _down_inputs(rng)
    got = moe.down_combine(act, w, chosen, weights, residual)
    block = torch.from_numpy(to_f32(act))
    g, u = block[:, :INNER], block[:, INNER:]
    a = (g / (1.0 + torch.exp(-g)) * u).double()
    rows = torch.from_numpy(to_f32(w)).double()[torch.from_numpy(chosen).long()]
    t = torch.einsum("kni,ki->kn", rows, a).float() * torch.from_numpy(weights)[:, None]
    d = t.to(torch.bfloat16).float()
    want = (d.sum(0).to(torch.bfloat16).float() + torch.from_numpy(to_f32(residual))).to(torch.bfloat16)
    want_bits = want.view(torch.int16).numpy().view(np.uint16)
    # torch's exp and the sum order of three terms may move a value by one ulp.
    assert ulp_distance(got, want_bits).max() <= 1
    assert (got == want_bits).mean() > 0.95


def test_down_combine_zero_weights_give_the_residual():
    rng = np.random.default_rng(3)
    act, w, chosen, _, residual = _down_inputs(rng)
    got = moe.down_combine(act, w, chosen, np.zeros(K, dtype=np.float32), residual)
    assert np.array_equal(got, residual)
    assert np.all(to_f32(moe.down_combine(act, w, chosen, np.zeros(K, np.float32), None)) == 0)


def test_down_combine_identity_matrix_returns_the_activation():
    rng = np.random.default_rng(4)
    act = from_float(rng.standard_normal((1, 2 * INNER)))
    eye = from_float(np.eye(INNER, dtype=np.float32))[None].repeat(2, axis=0)  # [2, I, I]
    got = moe.down_combine(act, eye, np.array([1], dtype=np.int32), np.array([1.0], np.float32), None)
    block = to_f32(act)[0]
    want = from_float(moe.swiglu_fp32(block[:INNER], block[INNER:]))
    assert np.array_equal(got, want)


def test_swiglu_fp32_special_values():
    g = np.array([0.0, -0.0, 30.0, -30.0, 100.0, -100.0], dtype=np.float32)
    u = np.ones_like(g)
    a = moe.swiglu_fp32(g, u)
    assert a[0] == 0.0 and a[1] == 0.0
    assert a[2] == np.float32(30.0) and a[4] == np.float32(100.0)   # sigmoid saturates to 1
    assert abs(a[3]) < 1e-11 and a[5] == 0.0                         # exp(100) -> inf -> g/inf


@pytest.mark.parametrize("kind", ["swapped", "no_weight", "no_residual"])
def test_planted_mistakes_fail(kind):
    rng = np.random.default_rng(5)
    act, w, chosen, weights, residual = _down_inputs(rng, k=4)
    weights = np.array([0.9, 1e-3, 5.0, 0.25], dtype=np.float32)
    good = moe.down_combine(act, w, chosen, weights, residual)
    if kind == "swapped":
        act = np.concatenate([act[:, INNER:], act[:, :INNER]], axis=1)
        bad = moe.down_combine(act, w, chosen, weights, residual)
    elif kind == "no_weight":
        bad = moe.down_combine(act, w, chosen, np.ones(4, np.float32), residual)
    else:
        bad = moe.down_combine(act, w, chosen, weights, None)
    assert not np.array_equal(good, bad)


def test_expert_order_only_moves_rounding():
    rng = np.random.default_rng(6)
    act, w, chosen, weights, residual = _down_inputs(rng, k=4)
    good = moe.down_combine(act, w, chosen, weights, residual)
    flipped = moe.down_combine(act[::-1].copy(), w, chosen[::-1].copy(), weights[::-1].copy(), residual)
    assert ulp_distance(good, flipped).max() <= 1

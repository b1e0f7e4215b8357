"""Pins the AddRMSNorm oracle (oracle/add_norm.py) with checks independent of its formula.

- the residual sum against torch's bf16 add (a library routine), bit for bit;
- the norm against torch's `F.rms_norm` in float64 with the declared rounding points
  applied around it, and against an fp64 closed form;
- the eps reach test of tests/test_kernel_add_rms_norm.py:133-144 (a tiny stream is where
  eps shows);
- invariants: unit weight gives unit RMS; scaling the input leaves the norm unchanged;
- planted mistakes (dropped eps, dropped weight, wrong mean, no intermediate rounding)
  each fail one of the checks above.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import add_norm
from oracle.bf16 import R, from_float, to_bf16, to_f32, ulp_distance

EPS = 1e-6


def _replica(rows, hidden, seed, *, checkpoint=False):
    rng = np.random.default_rng(seed)
    if checkpoint:
        # tests/test_kernel_add_rms_norm.py:34-43: a grown residual stream with outliers.
        x = rng.standard_normal((rows, hidden)) * 30.0
        x += rng.standard_normal((rows, hidden)) * 300.0 * (rng.uniform(size=(rows, hidden)) > 0.99)
        b = rng.standard_normal((rows, hidden)) * 3.0
        w = 1.0 + rng.standard_normal(hidden) * 0.2
    else:
        x = rng.standard_normal((rows, hidden))
        b = rng.standard_normal((rows, hidden))
        w = 1.0 + 0.1 * rng.standard_normal(hidden)
    return from_float(x), from_float(b), from_float(w)


def _torch_bf16(bits):
    return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)


def _independent_norm(s_bits, w_bits, eps):
    """torch F.rms_norm (fp64) for the normalised value, then the declared roundings."""
    s = torch.from_numpy(to_f32(s_bits).astype(np.float64))
    normed = F.rms_norm(s, (s.shape[-1],), eps=eps).numpy().astype(np.float32)
    return to_bf16(to_f32(w_bits) * R(normed))


@pytest.mark.parametrize("rows,hidden", [(1, 2560), (16, 2560), (3, 2048), (5, 2880)])
@pytest.mark.parametrize("checkpoint", [False, True])
def test_matches_library_chain(rows, hidden, checkpoint):
    x, b, w = _replica(rows, hidden, seed=rows + hidden, checkpoint=checkpoint)
    summed, normed = add_norm.add_rms_norm(x, b, w, EPS)
    torch_sum = (_torch_bf16(x) + _torch_bf16(b)).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(summed, torch_sum)
    independent = _independent_norm(summed, w, EPS)
    dist = ulp_distance(normed, independent)
    assert dist.max() <= 1
    assert np.mean(dist == 0) > 0.995


def test_close_to_fp64_closed_form():
    x, b, w = _replica(8, 2560, seed=3)
    summed, normed = add_norm.add_rms_norm(x, b, w, EPS)
    s = to_f32(summed).astype(np.float64)
    exact = to_f32(w) * s / np.sqrt(np.mean(s * s, axis=-1, keepdims=True) + EPS)
    # Two roundings to bf16 (the normalised value, then the product): <= 1 ulp each.
    assert ulp_distance(normed, to_bf16(exact.astype(np.float32))).max() <= 2


def test_eps_reaches_the_norm():
    x, b, w = _replica(2, 2048, seed=9)
    tiny_x = from_float(to_f32(x) * 1e-3)
    tiny_b = from_float(to_f32(b) * 1e-3)
    summed, with_big_eps = add_norm.add_rms_norm(tiny_x, tiny_b, w, 0.5)
    _, with_small_eps = add_norm.add_rms_norm(tiny_x, tiny_b, w, EPS)
    assert ulp_distance(with_big_eps, _independent_norm(summed, w, 0.5)).max() <= 1
    assert not np.array_equal(with_big_eps, with_small_eps)


def test_invariants():
    x, b, w = _replica(4, 2560, seed=5)
    one = from_float(np.ones(2560))
    summed, normed = add_norm.add_rms_norm(x, b, one, EPS)
    rms = np.sqrt(np.mean(to_f32(normed).astype(np.float64) ** 2, axis=-1))
    np.testing.assert_allclose(rms, 1.0, rtol=5e-3)
    # A power-of-two scale of the input is exact in bf16 and cancels in the norm.
    scaled = add_norm.rms_norm(from_float(to_f32(summed) * 4.0), w, 0.0)
    assert np.array_equal(scaled, add_norm.rms_norm(summed, w, 0.0))


def _planted(kind):
    def mutated(x_bits, b_bits, w_bits, eps):
        s_bits = to_bf16(to_f32(x_bits) + to_f32(b_bits))
        s = to_f32(s_bits)
        hidden = s.shape[-1]
        if kind == "no_eps":
            inv = 1.0 / np.sqrt(np.mean(s.astype(np.float64) ** 2, axis=-1, keepdims=True))
        elif kind == "wrong_mean":
            inv = 1.0 / np.sqrt(np.sum(s.astype(np.float64) ** 2, -1, keepdims=True) / (hidden - 1) + eps)
        else:
            inv = add_norm.inverse_rms(s, eps)
        inv = inv.astype(np.float32)
        if kind == "no_weight":
            return s_bits, to_bf16(R(s * inv))
        if kind == "no_rounding":
            return s_bits, to_bf16(to_f32(w_bits) * (s * inv))
        return s_bits, to_bf16(to_f32(w_bits) * R(s * inv))
    return mutated


@pytest.mark.parametrize("kind", ["no_eps", "wrong_mean", "no_weight", "no_rounding"])
def test_planted_mistakes_are_caught(kind):
    """Each plausible mistake fails at least one of the pinning checks above."""
    mutated = _planted(kind)
    caught = False
    for rows, hidden, seed in ((16, 2560, 1), (2, 2048, 9)):
        x, b, w = _replica(rows, hidden, seed)
        if kind == "no_eps":
            x, b = from_float(to_f32(x) * 1e-3), from_float(to_f32(b) * 1e-3)
            eps = 0.5
        else:
            eps = EPS
        summed, normed = mutated(x, b, w, eps)
        dist = ulp_distance(normed, _independent_norm(summed, w, eps))
        caught |= bool(dist.max() > 1 or np.mean(dist == 0) <= 0.995)
    assert caught

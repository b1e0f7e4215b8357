"""Pins the activation oracles (oracle/activations.py) independently of their formulas.

- the float64 -> bf16 rounding against exact rational arithmetic (fractions.Fraction):
  nearest bf16 neighbour, ties to even;
- SwiGLU against torch's own bf16 ops (sigmoid in float32 rounded to bf16, then bf16
  products), which can differ from the correctly rounded sigmoid only in the rare case
  where torch's float32 sigmoid sits on the wrong side of a bf16 midpoint;
- special values: g = 0 gives 0, large g gives bf16(g * u), very negative g gives a
  tiny value of the sign of -u;
- gate-softplus against torch's float64 softplus (no threshold), and its saturation
  arms and NaN propagation;
- planted mistakes (unrounded sigmoid, wrong sigmoid sign, a dropped dt_bias, the naive
  log(1 + exp(x)) that overflows) each fail one of the checks.
"""

from fractions import Fraction

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import activations as act
from oracle.bf16 import from_float, to_bf16, to_f32, ulp_distance


def _exact_bf16(x: float) -> int:
    """Round a finite double to bf16 by exact rational comparison (normal range)."""
    if x == 0:
        return 0x8000 if np.signbit(x) else 0
    sign = 0x8000 if x < 0 else 0
    ax = Fraction(abs(x))
    lo_bits = int(np.float32(abs(x)).view(np.uint32)) >> 16  # truncation candidate
    for cand in (lo_bits - 1, lo_bits, lo_bits + 1):
        lo = Fraction(float(np.array([cand << 16], np.uint32).view(np.float32)[0]))
        hi = Fraction(float(np.array([(cand + 1) << 16], np.uint32).view(np.float32)[0]))
        if lo <= ax < hi:
            mid = (lo + hi) / 2
            if ax < mid or (ax == mid and cand % 2 == 0):
                return sign | cand
            return sign | (cand + 1)
    raise AssertionError(x)


def test_f64_to_bf16_is_exactly_rounded():
    rng = np.random.default_rng(0)
    values = rng.standard_normal(4000) * 10.0 ** rng.integers(-30, 30, 4000)
    # Values one double ulp either side of bf16 midpoints: the double-rounding trap.
    mids = to_f32(rng.integers(0x3F80, 0x4080, 500).astype(np.uint16)).astype(np.float64) * (1 + 2.0**-9)
    values = np.concatenate([values, mids, np.nextafter(mids, 0), np.nextafter(mids, 10)])
    got = act.f64_to_bf16(values)
    want = np.array([_exact_bf16(float(v)) for v in values], dtype=np.uint16)
    assert np.array_equal(got, want)


def _gates(shape, seed):
    rng = np.random.default_rng(seed)
    return from_float(rng.standard_normal(shape)), from_float(rng.standard_normal(shape))


def _torch_swiglu(g_bits, u_bits):
    g = torch.from_numpy(g_bits.view(np.int16)).view(torch.bfloat16)
    u = torch.from_numpy(u_bits.view(np.int16)).view(torch.bfloat16)
    s = torch.sigmoid(g.float()).to(torch.bfloat16)
    return ((g * s) * u).view(torch.int16).numpy().view(np.uint16)


def test_swiglu_matches_torch_bf16_chain():
    g, u = _gates((64, 1024), seed=1)
    got = act.swiglu(g, u)
    want = _torch_swiglu(g, u)
    dist = ulp_distance(got, want)
    assert dist.max() <= 2 and np.mean(dist == 0) > 0.999


def test_sigmoid_is_correctly_rounded_against_exact_arithmetic():
    g = to_f32(from_float(np.random.default_rng(2).standard_normal(3000) * 4))
    got = act.sigmoid_bf16(g)
    from math import exp
    want = np.array([_exact_bf16(1.0 / (1.0 + exp(-float(x)))) for x in g], dtype=np.uint16)
    assert ulp_distance(got, want).max() == 0


def test_swiglu_special_values():
    g = from_float(np.array([0.0, 0.0, 20.0, -20.0, 30.0], np.float32))
    u = from_float(np.array([1.5, -2.0, 3.0, 2.0, -1.0], np.float32))
    y = to_f32(act.swiglu(g, u))
    assert y[0] == 0 and y[1] == 0
    assert y[2] == to_f32(to_bf16(np.float32(20.0 * 3.0)))
    assert -1e-6 < y[3] < 0
    assert y[4] == -30.0


def test_planted_swiglu_mistakes_fail():
    g, u = _gates((32, 1024), seed=3)
    want = _torch_swiglu(g, u)
    gf, uf = to_f32(g), to_f32(u)
    unrounded = to_bf16(to_f32(to_bf16(gf * (1 / (1 + np.exp(-gf))))) * uf)
    wrong_sign = to_bf16(to_f32(to_bf16(gf * to_f32(to_bf16(1 / (1 + np.exp(gf)))))) * uf)
    for planted in (unrounded, wrong_sign):
        dist = ulp_distance(planted, want)
        assert dist.max() > 2 or np.mean(dist == 0) <= 0.999


def _softplus_inputs(seed, rows=256, heads=32):
    rng = np.random.default_rng(seed)
    a = from_float(rng.standard_normal((rows, heads)))
    a_log = rng.uniform(0, 2.7, heads).astype(np.float32)
    dt_bias = (0.5 * rng.standard_normal(heads)).astype(np.float32)
    return a, a_log, dt_bias


def _torch_gate(a_bits, a_log, dt_bias):
    dt = torch.from_numpy(to_f32(a_bits) + dt_bias).double()
    sp = F.softplus(dt, beta=1.0, threshold=1e9)
    return (-torch.exp(torch.from_numpy(a_log).double()) * sp).numpy()


def test_gate_softplus_matches_torch_float64():
    a, a_log, dt_bias = _softplus_inputs(4)
    got = act.gate_softplus(a, a_log, dt_bias)
    np.testing.assert_allclose(got, _torch_gate(a, a_log, dt_bias), rtol=4e-7, atol=0)


def test_softplus_arms_and_nan():
    dt = np.array([np.inf, -np.inf, 40.0, -40.0, 0.0, -0.0, np.nan, 1e-30], np.float32)
    sp = act.softplus_f32(dt)
    assert sp[0] == np.inf and sp[1] == 0.0 and sp[2] == 40.0
    np.testing.assert_allclose(sp[3], np.exp(-40.0), rtol=1e-6)
    assert sp[4] == np.float32(np.log(2.0)) and sp[5] == np.float32(np.log(2.0))
    assert np.isnan(sp[6]) and sp[7] == np.float32(np.log(2.0))


def test_planted_softplus_mistakes_fail():
    a, a_log, dt_bias = _softplus_inputs(5)
    want = _torch_gate(a, a_log, dt_bias)
    no_bias = act.gate_softplus(a, a_log, np.zeros_like(dt_bias))
    assert not np.allclose(no_bias, want, rtol=1e-5)
    big = np.array([100.0], np.float32)
    with np.errstate(over="ignore"):
        naive = np.log(1 + np.exp(big.astype(np.float32) * 10))
    assert np.isinf(naive[0]) and np.isfinite(act.softplus_f32(big * 10)[0])

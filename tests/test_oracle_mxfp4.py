"""The MXFP4 routed-expert oracle (oracle/mxfp4.py) pinned without its own formula.

- The e2m1 table against the format's closed form (sign, two exponent bits, one mantissa
  bit, the subnormal e = 0), the nibble order by a hand-derived word, e8m0 factors by
  hand, and pack/codes as inverses.
- gate_up and down_combine against torch: the weights rebuilt from the integer codes by
  the closed form (no table) and a float64 matmul, then (a) the kernels' rounding points
  replayed in torch float32 ops (torch's exp and division), within the bf16 bar with 97%
  bit-identical, and (b) the reference's Core epilogue in torch bf16 ops
  (core/kernels/gate_up/default.py:59-78, down_combine/default.py:49-58), which rounds at
  other points (1.702 g to bf16 before the sigmoid), within a few percent.
  The clamp bites.
- Planted mistakes in the oracle (high nibble first, the scale exponent off by one, the
  projection bias dropped, the 1.702 factor dropped, the `up + 1` dropped) fail.
"""

import numpy as np
import pytest
import torch

from oracle import mxfp4
from oracle.bf16 import from_float, to_f32
from util import assert_bf16_close

HIDDEN, INNER, EXPERTS = 128, 64, 4


def _closed_form(code: int) -> float:
    sign = -1.0 if code & 8 else 1.0
    e, m = (code >> 1) & 3, code & 1
    return sign * (m / 2 if e == 0 else 2.0 ** (e - 1) * (1 + m / 2))


def test_e2m1_table_is_the_closed_form():
    assert [float(v) for v in mxfp4.E2M1] == [_closed_form(c) for c in range(16)]


def test_nibble_order_and_e8m0_by_hand():
    assert mxfp4.codes(np.array([0x87654321], dtype=np.uint32)).tolist() == [1, 2, 3, 4, 5, 6, 7, 8]
    assert mxfp4.scale_values(np.array([0, 1, 120, 127, 128], dtype=np.uint8)).tolist() == \
        [0.0, 2.0 ** -126, 2.0 ** -7, 1.0, 2.0]
    rng = np.random.default_rng(0)
    c = rng.integers(0, 16, size=(3, 5, 64))
    assert np.array_equal(mxfp4.codes(mxfp4.pack(c)), c)


class Case:
    def __init__(self, rows, features, seed, experts=EXPERTS):
        rng = np.random.default_rng(seed)
        self.c = rng.integers(0, 16, size=(experts, rows, features))
        self.s = rng.integers(118, 124, size=(experts, rows, features // 32)).astype(np.uint8)
        self.b = from_float(0.1 * rng.standard_normal((experts, rows)))
        self.stack = mxfp4.Stack(mxfp4.pack(self.c), self.s, self.b)

    def torch_matrix(self, e):
        c = torch.from_numpy(self.c[e]).long()
        sign = torch.where(c & 8 != 0, -1.0, 1.0).double()
        ex, m = ((c >> 1) & 3).double(), (c & 1).double()
        value = sign * torch.where(ex == 0, m / 2, torch.pow(2.0, ex - 1) * (1 + m / 2))
        scale = torch.pow(2.0, torch.from_numpy(self.s[e].astype(np.float64)) - 127)
        return value * scale.repeat_interleave(32, dim=-1)


def _bf16(t):
    return t.to(torch.bfloat16)


def _bits(t):
    return t.view(torch.int16).numpy().view(np.uint16)


def _torch_gate_up(case, x_bits, chosen, limit):
    """The Core chain: bf16 rows, bf16 ops."""
    x = torch.from_numpy(to_f32(x_bits)).double()
    rows = _bf16(torch.stack([case.torch_matrix(e) @ x for e in chosen]))
    fused = rows + _bf16(torch.from_numpy(to_f32(case.b[chosen])))
    gate, up = fused[:, 0::2], fused[:, 1::2]
    gate = torch.clamp(gate, max=limit)
    up = torch.clamp(up, -limit, limit)
    return _bits(gate * torch.sigmoid(1.702 * gate) * (up + 1))


def _torch_kernel_points(case, x_bits, chosen, limit):
    """The kernels' rounding points in torch float32 ops."""
    x = torch.from_numpy(to_f32(x_bits)).double()
    r = torch.stack([case.torch_matrix(e) @ x for e in chosen])
    fused = (r + torch.from_numpy(to_f32(case.b[chosen])).double()).float()
    g, u = _bf16(fused[:, 0::2]).float(), _bf16(fused[:, 1::2]).float()
    if limit is not None:
        g = _bf16(torch.clamp(g, max=limit)).float()
        u = _bf16(torch.clamp(u, -limit, limit)).float()
    sig = _bf16(1.0 / (1.0 + torch.exp(torch.tensor(-1.702, dtype=torch.float32) * g))).float()
    act = _bf16(g * sig).float()
    return _bits(_bf16(act * _bf16(u + 1.0).float()))


def test_gate_up_matches_torch_and_the_clamp_bites():
    case = Case(2 * INNER, HIDDEN, seed=1)
    x = from_float(3 * np.random.default_rng(2).standard_normal(HIDDEN))
    chosen = [3, 0, 2]
    for limit in (7.0, 0.25):
        got = mxfp4.gate_up(x, case.stack, chosen, limit)
        assert got.shape == (3, INNER)
        assert_bf16_close(got, _torch_kernel_points(case, x, chosen, limit), min_exact=0.97)
        # The Core chain rounds 1.702 g to bf16 (steps of 2^-5 near 5) before the sigmoid,
        # which moves a steep sigmoid by a few percent: the same function, looser.
        core = to_f32(_torch_gate_up(case, x, chosen, limit))
        np.testing.assert_allclose(to_f32(got), core, rtol=0.06, atol=0.02)
    assert not np.array_equal(mxfp4.gate_up(x, case.stack, chosen, 0.25),
                              mxfp4.gate_up(x, case.stack, chosen, None))


def _torch_down(case, act_bits, chosen, weights, residual_bits):
    act = torch.from_numpy(to_f32(act_bits)).double()
    down = _bf16(torch.stack([case.torch_matrix(e) @ act[j] for j, e in enumerate(chosen)]))
    down = down + _bf16(torch.from_numpy(to_f32(case.b[chosen])))
    out = (down * _bf16(torch.from_numpy(weights))[:, None]).sum(dim=0)
    return _bits(out + _bf16(torch.from_numpy(to_f32(residual_bits))))


def test_down_combine_matches_the_core_chain_and_zero_weights():
    case = Case(HIDDEN, INNER, seed=3)
    rng = np.random.default_rng(4)
    chosen = [1, 3, 0, 2]
    act = from_float(rng.standard_normal((4, INNER)))
    weights = to_f32(from_float(rng.dirichlet(np.ones(4))))
    residual = from_float(0.5 * rng.standard_normal(HIDDEN))
    got = mxfp4.down_combine(act, case.stack, chosen, weights, residual)
    # The Core chain rounds the row before the bias add; the kernels round once.
    assert_bf16_close(got, _torch_down(case, act, chosen, weights, residual), min_exact=0.8)
    zero = mxfp4.down_combine(act, case.stack, chosen, np.zeros(4, np.float32), residual)
    assert np.array_equal(to_f32(zero), to_f32(residual))


def _activation_without(part):
    """swiglu_oai with one term planted wrong."""
    def activation(g, u, limit):
        if limit is not None:
            g = mxfp4._T(np.minimum(g, np.float32(limit)))
            u = mxfp4._T(np.clip(u, np.float32(-limit), np.float32(limit)))
        k = np.float32(1.0 if part == "1.702" else -1.702 if part == "sign" else 1.702)
        sig = mxfp4._T(np.float32(1.0) / (np.float32(1.0) + np.exp(-k * g, dtype=np.float32)))
        one = np.float32(0.0 if part == "+1" else 1.0)
        return from_float(mxfp4._T(g * sig) * mxfp4._T(u + one))
    return activation


def _mutate(monkeypatch, name):
    if name == "high nibble first":
        real = mxfp4.codes
        monkeypatch.setattr(mxfp4, "codes", lambda w: np.flip(
            real(w).reshape(*real(w).shape[:-1], -1, 2), axis=-1).reshape(real(w).shape))
    elif name == "scale off by one":
        real = mxfp4.scale_values
        monkeypatch.setattr(mxfp4, "scale_values", lambda s: real(np.asarray(s, np.uint8) + 1))
    elif name == "bias dropped":
        real = mxfp4._slot
        monkeypatch.setattr(mxfp4, "_slot", lambda st, e: (real(st, e)[0], np.zeros_like(real(st, e)[1])))
    else:
        monkeypatch.setattr(mxfp4, "swiglu_oai", _activation_without(name))


@pytest.mark.parametrize("name", ["high nibble first", "scale off by one", "bias dropped", "1.702", "+1",
                                  "sign"])
def test_planted_gate_up_mistakes_fail(monkeypatch, name):
    case = Case(2 * INNER, HIDDEN, seed=5)
    x = from_float(np.random.default_rng(6).standard_normal(HIDDEN))
    want = _torch_kernel_points(case, x, [1, 2], 7.0)
    assert_bf16_close(mxfp4.gate_up(x, case.stack, [1, 2], 7.0), want, min_exact=0.97)
    _mutate(monkeypatch, name)
    with pytest.raises(AssertionError):
        assert_bf16_close(mxfp4.gate_up(x, case.stack, [1, 2], 7.0), want, min_exact=0.97)

"""The affine routed-expert oracle (oracle/affine.py) pinned without its own formula.

- The bit stream: hand-derived words for every width, including values that straddle two
  words (3, 5 and 6 bits); pack and unpack invert each other.
- Dequantization against a Python loop over the bit stream, one bit at a time.
- gate_up and down_combine against torch, fed the integer values directly (no decoding):
  float64 matmul of scale * q + bias, then the reference's Core epilogue in torch bf16 ops
  (core/kernels/gate_up/default.py:71-81, down_combine/default.py:49-58), within one bf16
  ulp; the clamp; the shared expert's slot; zero routing weights return the residual.
- Planted mistakes in the oracle (bits read MSB first, the zero point dropped, the
  group index off by one, the silu's sign flipped, the routing weight dropped) fail.
"""

import numpy as np
import pytest
import torch

from oracle import affine
from oracle.bf16 import from_float, to_f32, ulp_distance

HIDDEN, INNER, EXPERTS = 128, 64, 5


@pytest.mark.parametrize("bits,values,words", [
    (4, [1, 2, 3, 4, 5, 6, 7, 8], [0x87654321]),
    (8, [0x12, 0x34, 0x56, 0x78], [0x78563412]),
    (2, [3, 0, 1, 2] + [0] * 12, [0x93]),
    (3, [1, 2, 3, 4, 5, 6, 7] + [0] * 25, [0x001F58D1, 0, 0]),
    (3, [0] * 10 + [7] + [0] * 21, [0xC0000000, 0x1, 0]),     # bits 30..32
    (5, [0] * 6 + [31] + [0] * 25, [0xC0000000, 0x7, 0, 0, 0]),  # bits 30..34
    (6, [0] * 5 + [63] + [0] * 26, [0xC0000000, 0xF, 0, 0, 0, 0]),  # bits 30..35
])
def test_bit_stream_known_answers(bits, values, words):
    assert affine.pack(np.array(values), bits).tolist() == words
    assert affine.unpack(np.array(words, dtype=np.uint32), bits).tolist() == values


@pytest.mark.parametrize("bits", affine.WIDTHS)
def test_pack_unpack_round_trip(bits):
    rng = np.random.default_rng(bits)
    q = rng.integers(0, 1 << bits, size=(3, 7, 64))
    packed = affine.pack(q, bits)
    assert packed.shape == (3, 7, 64 * bits // 32) and packed.dtype == np.uint32
    assert np.array_equal(affine.unpack(packed, bits), q)


def _stack_from_q(q, scales, biases, group, bits):
    return affine.Stack(affine.pack(q, bits), scales, biases, group, bits)


@pytest.mark.parametrize("bits", affine.WIDTHS)
def test_dequantize_matches_a_bitwise_loop(bits):
    rng = np.random.default_rng(10 + bits)
    out, inp, group = 2, 64, 32
    q = rng.integers(0, 1 << bits, size=(out, inp))
    s = from_float(0.01 + 0.1 * rng.random((out, inp // group)))
    b = from_float(rng.standard_normal((out, inp // group)))
    stack = _stack_from_q(q, s, b, group, bits)
    got = affine.dequantize(stack)
    words = stack.weight.tolist()
    for o in range(out):
        for j in range(inp):
            value = 0
            for i in range(bits):
                bit = j * bits + i
                value |= ((words[o][bit // 32] >> (bit % 32)) & 1) << i
            want = float(to_f32(s[o, j // group])) * value + float(to_f32(b[o, j // group]))
            assert got[o, j] == want


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("group", affine.GROUPS)
def test_quantize_reconstructs_within_a_step(bits, group):
    rng = np.random.default_rng(bits * group)
    w = 0.05 * rng.standard_normal((3, 8, 256))
    stack = affine.quantize(w, group, bits)
    step = np.repeat(to_f32(stack.scales).astype(np.float64), group, axis=-1)
    assert np.all(np.abs(affine.dequantize(stack) - w) <= step * 1.01 + 1e-6)


class Case:
    """A stack built from known integers, so torch can use them without decoding."""

    def __init__(self, bits, group, out, inp, seed, experts=EXPERTS):
        rng = np.random.default_rng(seed)
        self.q = rng.integers(0, 1 << bits, size=(experts, out, inp))
        self.s = from_float((0.5 / (1 << bits)) * (0.5 + rng.random((experts, out, inp // group))) / np.sqrt(inp))
        self.b = from_float(-0.25 / np.sqrt(inp) * rng.random((experts, out, inp // group)))
        self.stack = _stack_from_q(self.q, self.s, self.b, group, bits)
        self.group = group

    def torch_matrix(self, e):
        s = torch.from_numpy(to_f32(self.s[e])).double().repeat_interleave(self.group, dim=-1)
        b = torch.from_numpy(to_f32(self.b[e])).double().repeat_interleave(self.group, dim=-1)
        return s * torch.from_numpy(self.q[e]).double() + b


def _torch_gate_up(case, x_bits, chosen, limit=None):
    x = torch.from_numpy(to_f32(x_bits)).double()
    rows = torch.stack([case.torch_matrix(e) @ x for e in chosen]).to(torch.bfloat16)
    pairs = rows.reshape(len(chosen), -1, 2)
    gate, up = pairs[..., 0], pairs[..., 1]
    if limit is not None:
        gate = torch.clamp(gate, max=limit)
        up = torch.clamp(up, -limit, limit)
    return (gate * torch.sigmoid(gate) * up).view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("bits", affine.WIDTHS)
@pytest.mark.parametrize("group", affine.GROUPS)
def test_gate_up_matches_torch(bits, group):
    case = Case(bits, group, 2 * INNER, HIDDEN, seed=bits + group)
    x = from_float(np.random.default_rng(3).standard_normal(HIDDEN))
    chosen = [3, 0, 4]
    got = affine.gate_up(x, case.stack, chosen)
    want = _torch_gate_up(case, x, chosen)
    assert got.shape == (3, INNER)
    assert ulp_distance(got, want).max() <= 1
    assert (got == want).mean() > 0.98


def test_gate_up_clamp_bites_and_matches_torch():
    case = Case(4, 64, 2 * INNER, HIDDEN, seed=5)
    x = from_float(4 * np.random.default_rng(4).standard_normal(HIDDEN))
    limit = 0.25
    got = affine.gate_up(x, case.stack, [1, 2], limit=limit)
    assert ulp_distance(got, _torch_gate_up(case, x, [1, 2], limit)).max() <= 1
    assert not np.array_equal(got, affine.gate_up(x, case.stack, [1, 2]))


def test_shared_slot_reads_its_own_leaf():
    case = Case(4, 64, 2 * INNER, HIDDEN, seed=6)
    other = Case(3, 32, 2 * INNER, HIDDEN, seed=7, experts=1)
    shared = affine.Stack(other.stack.weight[0], other.s[0], other.b[0], 32, 3)
    x = from_float(np.random.default_rng(8).standard_normal(HIDDEN))
    got = affine.gate_up(x, case.stack, [2, 99], shared=shared)   # the last index is not read
    assert np.array_equal(got[0], affine.gate_up(x, case.stack, [2])[0])
    assert np.array_equal(got[1], affine.gate_up(x, other.stack, [0])[0])


def _torch_down(case, act_bits, chosen, weights, residual_bits):
    act = torch.from_numpy(to_f32(act_bits)).double()
    down = torch.stack([case.torch_matrix(e) @ act[j] for j, e in enumerate(chosen)]).to(torch.bfloat16)
    out = (down * torch.from_numpy(weights).to(torch.bfloat16)[:, None]).sum(dim=0)
    out = out + torch.from_numpy(to_f32(residual_bits)).to(torch.bfloat16)
    return out.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("bits", affine.WIDTHS)
def test_down_combine_matches_the_core_chain(bits):
    case = Case(bits, 64, HIDDEN, INNER, seed=20 + bits)
    rng = np.random.default_rng(21)
    chosen = [4, 1, 0, 2]
    act = from_float(rng.standard_normal((4, INNER)))
    weights = to_f32(from_float(rng.dirichlet(np.ones(4))))      # bf16-valued router weights
    residual = from_float(0.5 * rng.standard_normal(HIDDEN))
    got = affine.down_combine(act, case.stack, chosen, weights, residual)
    want = _torch_down(case, act, chosen, weights, residual)
    # The Core chain rounds the per-expert products and the sum at other points.
    assert ulp_distance(got, want).max() <= 2
    assert (got == want).mean() > 0.9


def test_down_combine_zero_weights_return_the_residual():
    case = Case(4, 32, HIDDEN, INNER, seed=30)
    rng = np.random.default_rng(31)
    residual = from_float(rng.standard_normal(HIDDEN))
    act = from_float(rng.standard_normal((2, INNER)))
    got = affine.down_combine(act, case.stack, [0, 3], np.zeros(2, np.float32), residual)
    assert np.array_equal(to_f32(got), to_f32(residual))


def _mutations(monkeypatch, name):
    if name == "msb-first":
        real = affine.unpack
        monkeypatch.setattr(affine, "unpack", lambda w, bits: real(w, bits)[..., ::-1].copy())
    elif name == "zero point dropped":
        real = affine.dequantize
        monkeypatch.setattr(affine, "dequantize", lambda st: real(affine.Stack(
            st.weight, st.scales, np.zeros_like(st.biases), st.group, st.bits)))
    elif name == "group off by one":
        real = affine.dequantize
        monkeypatch.setattr(affine, "dequantize", lambda st: real(affine.Stack(
            st.weight, np.roll(st.scales, 1, axis=-1), st.biases, st.group, st.bits)))
    elif name == "silu sign":
        monkeypatch.setattr(affine, "sigmoid_bf16",
                            lambda g: to_f32(from_float(1.0 / (1.0 + np.exp(np.asarray(g, np.float64))))))


@pytest.mark.parametrize("name", ["msb-first", "zero point dropped", "group off by one", "silu sign"])
def test_planted_gate_up_mistakes_fail(monkeypatch, name):
    case = Case(4, 32, 2 * INNER, HIDDEN, seed=40)
    x = from_float(np.random.default_rng(41).standard_normal(HIDDEN))
    want = _torch_gate_up(case, x, [1, 3])
    _mutations(monkeypatch, name)
    got = affine.gate_up(x, case.stack, [1, 3])
    assert ulp_distance(got, want).max() > 2


def test_planted_down_mistake_fails(monkeypatch):
    case = Case(4, 64, HIDDEN, INNER, seed=50)
    rng = np.random.default_rng(51)
    act = from_float(rng.standard_normal((2, INNER)))
    weights = to_f32(from_float(np.array([0.3, 0.7])))
    residual = from_float(0.1 * rng.standard_normal(HIDDEN))
    want = _torch_down(case, act, [2, 4], weights, residual)
    got = affine.down_combine(act, case.stack, [2, 4], np.ones(2, np.float32), residual)
    assert ulp_distance(got, want).max() > 2

"""The NVFP4 routed-expert oracle (oracle/nvfp4.py) pinned without its own formula.

- The e4m3 table against mlx's own route (the magnitude bits placed in an IEEE half and
  scaled by 2^8, core/kernels/shared/nvfp4/qmoe.py:22-37) for all 256 bytes, and by hand
  (0, the smallest subnormal, the smallest normal, 1, 448, 480 for 0x7F, signs).
- gate_up and down_combine against torch: the weights rebuilt from the integer codes by
  the e2m1 closed form and the half route, a float64 matmul, the kernels' rounding points
  replayed in torch float32 ops (torch's exp and division), within the bf16 bar with 97%
  bit-identical; the reference's Core epilogue in torch bf16 ops within a few percent.
- Planted mistakes in the oracle (the scale's sign dropped, groups of 32, the high nibble
  first, the silu's sign, the up rounding skipped) fail.
"""

import numpy as np
import pytest
import torch

from oracle import nvfp4
from oracle.bf16 import from_float, to_f32
from util import assert_bf16_close

HIDDEN, INNER, EXPERTS = 128, 64, 4


def _half_route(byte: int) -> float:
    magnitude = np.array([(byte & 0x7F) << 7], dtype=np.uint16).view(np.float16)[0]
    value = float(magnitude) * 256.0
    return -value if byte & 0x80 else value


def test_e4m3_table_is_mlx_half_route_and_by_hand():
    assert [float(v) for v in nvfp4.E4M3] == [_half_route(b) for b in range(256)]
    by_hand = {0x00: 0.0, 0x01: 2.0 ** -9, 0x07: 7 * 2.0 ** -9, 0x08: 2.0 ** -6, 0x38: 1.0,
               0x3C: 1.5, 0x7E: 448.0, 0x7F: 480.0, 0xB8: -1.0, 0xFF: -480.0}
    for byte, value in by_hand.items():
        assert nvfp4.E4M3[byte] == value, hex(byte)
    assert np.signbit(nvfp4.E4M3[0x80])


def _closed_e2m1(c):
    sign = torch.where(c & 8 != 0, -1.0, 1.0).double()
    ex, m = ((c >> 1) & 3).double(), (c & 1).double()
    return sign * torch.where(ex == 0, m / 2, torch.pow(2.0, ex - 1) * (1 + m / 2))


class Case:
    def __init__(self, rows, features, seed, experts=EXPERTS):
        rng = np.random.default_rng(seed)
        self.c = rng.integers(0, 16, size=(experts, rows, features))
        # positive scales near 2^-4 with random mantissas, and a few negative ones
        self.s = (rng.integers(0x18, 0x28, size=(experts, rows, features // 16))
                  | (rng.random((experts, rows, features // 16)) < 0.1) * 0x80).astype(np.uint8)
        self.stack = nvfp4.Stack(nvfp4.pack(self.c), self.s)

    def torch_matrix(self, e):
        scale = torch.tensor([_half_route(int(b)) for b in self.s[e].reshape(-1)],
                             dtype=torch.float64).reshape(self.s[e].shape)
        return _closed_e2m1(torch.from_numpy(self.c[e]).long()) * scale.repeat_interleave(16, dim=-1)


def _bf16(t):
    return t.to(torch.bfloat16)


def _bits(t):
    return t.view(torch.int16).numpy().view(np.uint16)


def _torch_kernel_points(case, x_bits, chosen):
    x = torch.from_numpy(to_f32(x_bits)).double()
    r = torch.stack([case.torch_matrix(e) @ x for e in chosen]).float()
    g, u = _bf16(r[:, 0::2]).float(), _bf16(r[:, 1::2]).float()
    sig = _bf16(1.0 / (1.0 + torch.exp(-g))).float()
    return _bits(_bf16(_bf16(g * sig).float() * u))


def _torch_core(case, x_bits, chosen):
    x = torch.from_numpy(to_f32(x_bits)).double()
    fused = _bf16(torch.stack([case.torch_matrix(e) @ x for e in chosen]))
    gate, up = fused[:, 0::2], fused[:, 1::2]
    return _bits(gate * torch.sigmoid(gate) * up)


def test_gate_up_matches_torch():
    case = Case(2 * INNER, HIDDEN, seed=1)
    x = from_float(2 * np.random.default_rng(2).standard_normal(HIDDEN))
    chosen = [3, 0, 2]
    got = nvfp4.gate_up(x, case.stack, chosen)
    assert got.shape == (3, INNER)
    assert_bf16_close(got, _torch_kernel_points(case, x, chosen), min_exact=0.97)
    np.testing.assert_allclose(to_f32(got), to_f32(_torch_core(case, x, chosen)), rtol=0.03, atol=0.02)


def _torch_down(case, act_bits, chosen, weights, residual_bits):
    act = torch.from_numpy(to_f32(act_bits)).double()
    down = _bf16(torch.stack([case.torch_matrix(e) @ act[j] for j, e in enumerate(chosen)]).float())
    terms = _bf16(down.float() * torch.from_numpy(weights)[:, None]).float()
    acc = terms[0].clone()
    for row in terms[1:]:
        acc = acc + row
    return _bits(_bf16(_bf16(acc).float() + torch.from_numpy(to_f32(residual_bits))))


def test_down_combine_matches_torch_and_zero_weights():
    case = Case(HIDDEN, INNER, seed=3)
    rng = np.random.default_rng(4)
    chosen = [1, 3, 0, 2]
    act = from_float(rng.standard_normal((4, INNER)))
    weights = rng.dirichlet(np.ones(4)).astype(np.float32)
    residual = from_float(0.5 * rng.standard_normal(HIDDEN))
    got = nvfp4.down_combine(act, case.stack, chosen, weights, residual)
    assert_bf16_close(got, _torch_down(case, act, chosen, weights, residual), min_exact=0.97)
    zero = nvfp4.down_combine(act, case.stack, chosen, np.zeros(4, np.float32), residual)
    assert np.array_equal(to_f32(zero), to_f32(residual))


def _mutate(monkeypatch, name):
    if name == "scale sign dropped":
        monkeypatch.setattr(nvfp4, "E4M3", np.abs(nvfp4.E4M3))
    elif name == "groups of 32":
        monkeypatch.setattr(nvfp4, "dequantize", lambda st: nvfp4.E2M1[nvfp4.codes(st.weight)] * np.repeat(
            np.repeat(nvfp4.scale_values(st.scales)[..., ::2], 2, axis=-1), 16, axis=-1))
    elif name == "high nibble first":
        real = nvfp4.codes
        monkeypatch.setattr(nvfp4, "codes", lambda w: np.flip(
            real(w).reshape(*real(w).shape[:-1], -1, 2), axis=-1).reshape(real(w).shape))
    elif name == "silu sign":
        def swiglu(g, u):
            sig = nvfp4._T(np.float32(1.0) / (np.float32(1.0) + np.exp(g, dtype=np.float32)))
            return from_float(nvfp4._T(g * sig) * u)
        monkeypatch.setattr(nvfp4, "swiglu", swiglu)


@pytest.mark.parametrize("name", ["scale sign dropped", "groups of 32", "high nibble first", "silu sign"])
def test_planted_mistakes_fail(monkeypatch, name):
    case = Case(2 * INNER, HIDDEN, seed=5)
    x = from_float(np.random.default_rng(6).standard_normal(HIDDEN))
    want = _torch_kernel_points(case, x, [1, 2])
    assert_bf16_close(nvfp4.gate_up(x, case.stack, [1, 2]), want, min_exact=0.97)
    _mutate(monkeypatch, name)
    with pytest.raises(AssertionError):
        assert_bf16_close(nvfp4.gate_up(x, case.stack, [1, 2]), want, min_exact=0.97)


# ---- the packed form: the halved plane's certificate and the bf16 epilogue ------------
#
# core/kernels/down_combine/nvfp4_packed.py reads a halved group-32 plane
# (shared/nvfp4/packed.py:126-164) and ends in a bf16 chain. Pinned here:
# - the certificate and the halved plane's layout by hand;
# - that reading the halved plane the reference's way (byte `lane >> 1` of the row's
#   halved bytes, the header's byte for the second group of expert 0's row 0) decodes
#   exactly what the checkpoint's group-16 plane decodes, for certified planes;
# - down_combine_shared bit for bit against the reference test's own composition
#   (tests/test_kernel_nvfp4_fused_down_residual.py:88-118) restated in torch: float64
#   projections rounded to bf16, then `routed * w + total` and
#   `residual + (total + shared)` as bf16 tensor ops;
# - and that the comparison tells apart the mistakes an oracle could make (the shared
#   slot weighted, an fp32 running sum, the weights not rounded to bf16, the slots summed
#   in reverse).


def _paired_case(rows, features, seed, experts=EXPERTS):
    case = Case(rows, features, seed, experts)
    case.s = case.s & 0x7F                   # the halved plane refuses sign bits
    case.s[..., 1::2] = case.s[..., 0::2]    # mlx's quantizer writes both halves of a span alike
    case.stack = nvfp4.Stack(case.stack.weight, case.s)
    return case


def test_halved_scales_by_hand():
    plane = np.array([[[5, 5, 9, 9], [7, 7, 3, 3]]], np.uint8)
    got = nvfp4.halved_scales(plane)
    assert got.shape == (nvfp4.PATCH_BYTES + 4,)
    assert got[:2].tolist() == [5, 0] and not got[1:nvfp4.PATCH_BYTES].any()
    assert got[nvfp4.PATCH_BYTES:].tolist() == [5, 9, 7, 3]
    first = plane.copy()
    first[0, 0, 1] = 11          # flat pair 0 may differ: its odd byte goes to the header
    assert nvfp4.halved_scales(first)[0] == 11
    other = plane.copy()
    other[0, 1, 3] = 4           # any other unequal pair refuses the plane
    assert nvfp4.halved_scales(other) is None
    signed = plane.copy()
    signed[0, 1, :2] = 0x90      # so does a sign bit
    assert nvfp4.halved_scales(signed) is None


def _halved_read(halved, codes, expert, row_count, features, patched):
    """Expert `expert`'s [rows, features] weights read through the halved plane as
    nvfp4_packed.py:60-105 addresses it (one byte per 32 values; lane 1 of row 0 takes
    the header's byte when `patched`)."""
    per_row = features // 32
    out = np.zeros((row_count, features))
    for r in range(row_count):
        for j in range(features):
            at = nvfp4.PATCH_BYTES + (expert * row_count + r) * per_row + j // 32
            byte = halved[0] if patched and r == 0 and 16 <= j < 32 else halved[at]
            out[r, j] = nvfp4.E2M1[codes[expert, r, j]] * nvfp4.E4M3[byte]
    return out


def test_halved_read_decodes_what_the_group16_plane_decodes():
    case = _paired_case(8, 64, seed=11, experts=3)
    case.s[0, 0, 1] = 0x33       # the quantizer's first span, restored from the header
    stack = nvfp4.Stack(case.stack.weight, case.s)
    halved = nvfp4.halved_scales(case.s)
    assert halved is not None
    codes = nvfp4.codes(stack.weight)
    for e in range(3):
        want = nvfp4.dequantize(nvfp4.Stack(stack.weight[e], stack.scales[e]))
        assert np.array_equal(_halved_read(halved, codes, e, 8, 64, patched=e == 0), want)


def _packed_inputs(seed, tokens, k, hidden=HIDDEN, inner=512):
    rng = np.random.default_rng(seed)
    case = _paired_case(hidden, inner, seed, experts=6)
    shared = _paired_case(hidden, inner, seed + 1, experts=1)
    act = from_float(rng.standard_normal((tokens, k + 1, inner)))
    chosen = np.concatenate([rng.integers(0, 6, size=(tokens, k)), np.full((tokens, 1), 99)], axis=1)
    weights = np.concatenate([(rng.random((tokens, k)) * 2.5).astype(np.float32),
                              np.full((tokens, 1), 7.0, np.float32)], axis=1)
    residual = from_float(rng.standard_normal((tokens, hidden)))
    return case, shared, act, chosen, weights, residual


def _torch_packed(case, shared, act_bits, chosen, weights, residual_bits, *, weigh_shared=False,
                  fp32_total=False, unrounded_weights=False, reverse=False):
    out = []
    tokens, slots = act_bits.shape[:2]
    k = slots - 1
    for t in range(tokens):
        act = torch.from_numpy(to_f32(act_bits[t])).double()
        routed = _bf16(torch.stack([case.torch_matrix(e) @ act[j] for j, e in enumerate(chosen[t, :k])]).float())
        unrouted = _bf16((shared.torch_matrix(0) @ act[k]).float())
        w = torch.from_numpy(weights[t, :k])
        w = w if unrounded_weights else _bf16(w)
        order = range(k - 1, -1, -1) if reverse else range(k)
        if fp32_total:
            total = torch.zeros(routed.shape[1])
            for s in order:
                total = total + _bf16(routed[s].float() * w[s].float()).float()
            total = _bf16(total)
        else:
            total = torch.zeros(routed.shape[1], dtype=torch.bfloat16)
            for s in order:
                total = _bf16(routed[s].float() * w[s].float()) + total
        if weigh_shared:
            unrouted = _bf16(unrouted.float() * float(weights[t, k]))
        residual = _bf16(torch.from_numpy(to_f32(residual_bits[t])))
        out.append(_bits(residual + (total + unrouted)))
    return np.stack(out)


@pytest.mark.parametrize("tokens,k", [(1, 4), (2, 4), (3, 8)])
def test_down_combine_shared_matches_the_reference_composition(tokens, k):
    case, shared, act, chosen, weights, residual = _packed_inputs(20 + tokens, tokens, k)
    got = nvfp4.down_combine_shared(act, case.stack, nvfp4.Stack(shared.stack.weight[0], shared.s[0]),
                                    chosen, weights, residual)
    assert got.shape == (tokens, HIDDEN)
    assert np.array_equal(got, _torch_packed(case, shared, act, chosen, weights, residual))


@pytest.mark.parametrize("mistake", ["weigh_shared", "fp32_total", "unrounded_weights", "reverse"])
def test_down_combine_shared_comparison_tells_mistakes_apart(mistake):
    case, shared, act, chosen, weights, residual = _packed_inputs(30, 3, 8)
    got = nvfp4.down_combine_shared(act, case.stack, nvfp4.Stack(shared.stack.weight[0], shared.s[0]),
                                    chosen, weights, residual)
    wrong = _torch_packed(case, shared, act, chosen, weights, residual, **{mistake: True})
    assert not np.array_equal(got, wrong)

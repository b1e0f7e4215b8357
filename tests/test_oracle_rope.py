"""Pins the QK-norm + RoPE oracle (oracle/rope.py) with checks independent of its formula.

- the angle table against the closed form cos/sin(pos * base^(-i/P)) in float64;
- position 0 is the identity rotation (cos 1, sin 0): the output is the norm, bit for bit;
- the rotation against torch's complex multiplication (x1 + i x2) * (cos + i sin) in
  float64, which fixes the sign convention and the (p, p+P) pairing independently;
- rotations preserve each pair's length; the partial-rotary tail is the norm verbatim and
  ignores the angles (tests/test_kernel_qk_norm_rope.py:258-300);
- mscale: a power of two scales the rotary section exactly and leaves the tail;
- the epilogue's in-kernel angle formula (core/kernels/qkv_rope/epilogue.py:57-63)
  restated with torch's float64 exp2/cos/sin gives the same float32 bits, and stays
  within the fp32 angle error of the closed form;
- planted mistakes (swapped cos/sin, flipped sign, off-by-one partner, frozen position)
  each fail one of the checks.
"""

import math

import numpy as np
import pytest
import torch

from oracle import rope
from oracle.add_norm import rms_norm
from oracle.bf16 import R, from_float, to_bf16, to_f32, ulp_distance

EPS = 1e-6
MSCALE = 1.3465735912322998


def _inputs(length, heads, head_dim, seed):
    rng = np.random.default_rng(seed)
    raw = from_float(rng.standard_normal((length, heads, head_dim)))
    weight = from_float(1.0 + 0.1 * rng.standard_normal(head_dim))
    return raw, weight


def _complex_reference(raw, weight, cos, sin, pairs, mscale=1.0):
    """torch complex rotation of the (pinned) norm; [H, T, D] bf16 bits."""
    normed = rms_norm(raw, weight, EPS)
    n = torch.from_numpy(to_f32(normed))
    scale = torch.tensor(mscale, dtype=torch.float32).to(torch.bfloat16)
    first = (n[..., :pairs].to(torch.bfloat16) * scale).double()
    second = (n[..., pairs : 2 * pairs].to(torch.bfloat16) * scale).double()
    turn = torch.complex(torch.from_numpy(cos).double(), torch.from_numpy(sin).double())[:, None, :]
    z = torch.complex(first, second) * turn
    rotated = np.concatenate(
        [to_bf16(z.real.float().numpy()), to_bf16(z.imag.float().numpy()), normed[..., 2 * pairs :]],
        axis=-1,
    )
    return rotated.transpose(1, 0, 2)


def test_table_matches_closed_form():
    pairs, base, first = 64, 1e6, 36_000
    cos, sin = rope.angle_table(900, pairs, base, first=first)
    pos = np.arange(first, first + 900, dtype=np.float64)[:, None]
    theta = pos * np.array([base ** (-i / pairs) for i in range(pairs)])[None, :]
    assert np.abs(cos - np.cos(theta)).max() < 2e-7
    assert np.abs(sin - np.sin(theta)).max() < 2e-7


def test_position_zero_is_identity():
    raw, weight = _inputs(1, 6, 128, seed=1)
    cos, sin = rope.angle_table(4, 64, 1e6)
    out = rope.norm_rotate(raw, weight, cos[:1], sin[:1], EPS, 64)
    assert np.array_equal(out.transpose(1, 0, 2), rms_norm(raw, weight, EPS))


@pytest.mark.parametrize("head_dim,pairs", [(128, 64), (128, 32), (64, 16), (256, 128)])
@pytest.mark.parametrize("mscale", [1.0, MSCALE])
def test_matches_complex_rotation(head_dim, pairs, mscale):
    raw, weight = _inputs(9, 5, head_dim, seed=head_dim + pairs)
    cos, sin = rope.angle_table(40, pairs, 1e6)
    out = rope.norm_rotate(raw, weight, cos[20:29], sin[20:29], EPS, pairs, mscale)
    want = _complex_reference(raw, weight, cos[20:29], sin[20:29], pairs, mscale)
    dist = ulp_distance(out, want)
    assert dist.max() <= 1 and np.mean(dist == 0) > 0.99


def test_rotation_preserves_pair_length():
    raw, weight = _inputs(8, 4, 128, seed=3)
    cos, sin = rope.angle_table(2000, 64, 1e6)
    out = to_f32(rope.norm_rotate(raw, weight, cos[1990:1998], sin[1990:1998], EPS, 64)).astype(np.float64)
    n = to_f32(rms_norm(raw, weight, EPS)).transpose(1, 0, 2).astype(np.float64)
    before = n[..., :64] ** 2 + n[..., 64:] ** 2
    after = out[..., :64] ** 2 + out[..., 64:] ** 2
    np.testing.assert_allclose(after, before, rtol=2e-2, atol=1e-4)


def test_partial_tail_is_norm_verbatim_and_ignores_angles():
    raw, weight = _inputs(5, 4, 128, seed=13)
    a_cos, a_sin = rope.angle_table(8, 32, 1e6)
    b_cos, b_sin = rope.angle_table(8, 32, 1e4)
    a = rope.norm_rotate(raw, weight, a_cos[3:], a_sin[3:], EPS, 32, MSCALE)
    b = rope.norm_rotate(raw, weight, b_cos[3:], b_sin[3:], EPS, 32, MSCALE)
    normed = rms_norm(raw, weight, EPS).transpose(1, 0, 2)
    assert np.array_equal(a[..., 64:], normed[..., 64:])
    assert np.array_equal(a[..., 64:], b[..., 64:])
    assert not np.array_equal(a[..., :64], b[..., :64])


def test_power_of_two_mscale_scales_exactly():
    raw, weight = _inputs(6, 4, 128, seed=8)
    cos, sin = rope.angle_table(16, 32, 1e6)
    one = rope.norm_rotate(raw, weight, cos[10:], sin[10:], EPS, 32, 1.0)
    two = rope.norm_rotate(raw, weight, cos[10:], sin[10:], EPS, 32, 2.0)
    assert np.array_equal(to_f32(two[..., :64]), 2.0 * to_f32(one[..., :64]))
    assert np.array_equal(two[..., 64:], one[..., 64:])


def test_epilogue_angles_agree_with_torch_restatement():
    positions = np.array([0, 1, 137, 4095, 32767, 36862])
    cos, sin = rope.epilogue_angles(positions, 64, 1e6)
    d = torch.arange(64, dtype=torch.float32) / 64
    frequency = torch.exp2((-d * torch.tensor(math.log2(1e6), dtype=torch.float32)).double()).float()
    angle = (torch.tensor(positions, dtype=torch.float32)[:, None] * frequency[None, :]).double()
    assert np.array_equal(cos, torch.cos(angle).float().numpy())
    assert np.array_equal(sin, torch.sin(angle).float().numpy())
    exact = positions[:, None] * (1e6 ** (-np.arange(64) / 64))[None, :]
    # fp32 angle error grows with the position (an fp32 ulp of pos * frequency).
    bound = positions[:, None] * 2.0**-22 + 1e-6
    assert (np.abs(cos - np.cos(exact)) <= bound).all()


def test_epilogue_is_the_table_kernel_on_its_own_angles():
    rng = np.random.default_rng(4)
    hq, hkv, d, length, offset = 4, 2, 128, 6, 4090
    fused = from_float(rng.standard_normal((length, (hq + 2 * hkv) * d)))
    qw, kw = from_float(1 + 0.1 * rng.standard_normal(d)), from_float(1 + 0.1 * rng.standard_normal(d))
    q, k = rope.rope_epilogue(fused, hq, hkv, d, qw, kw, offset, 1e6, EPS)
    cos, sin = rope.epilogue_angles(np.arange(offset + length), 64, 1e6)
    raw_q = fused[:, : hq * d].reshape(length, hq, d)
    raw_k = fused[:, hq * d : (hq + hkv) * d].reshape(length, hkv, d)
    tq, tk = rope.qk_norm_rope(raw_q, raw_k, qw, kw, cos, sin, offset, EPS, 64)
    assert np.array_equal(q, tq) and np.array_equal(k, tk)


def _planted(kind):
    def mutated(raw, weight, cos, sin, eps, pairs, mscale=1.0):
        n = to_f32(rms_norm(raw, weight, eps))
        a, b = n[..., :pairs], n[..., pairs : 2 * pairs]
        c, s = cos[:, None, :], sin[:, None, :]
        if kind == "swap":
            c, s = s, c
        if kind == "sign":
            o1, o2 = a * c + b * s, -a * s + b * c
        elif kind == "partner":
            b = np.roll(b, 1, axis=-1)
            o1, o2 = a * c - b * s, a * s + b * c
        else:
            if kind == "frozen":
                c, s = np.broadcast_to(c[:1], c.shape), np.broadcast_to(s[:1], s.shape)
            o1, o2 = a * c - b * s, a * s + b * c
        out = np.concatenate([to_bf16(o1), to_bf16(o2), to_bf16(n[..., 2 * pairs :])], -1)
        return out.transpose(1, 0, 2)
    return mutated


@pytest.mark.parametrize("kind", ["swap", "sign", "partner", "frozen"])
def test_planted_mistakes_fail_the_complex_check(kind):
    raw, weight = _inputs(9, 5, 128, seed=5)
    cos, sin = rope.angle_table(40, 64, 1e6)
    out = _planted(kind)(raw, weight, cos[20:29], sin[20:29], EPS, 64)
    want = _complex_reference(raw, weight, cos[20:29], sin[20:29], 64)
    assert ulp_distance(out, want).max() > 2


# ---- the atlas in Laguna's fp32 order ---------------------------------------------------


def test_laguna_inverse_row_against_fp32_libraries():
    """The fp32 power against torch's and numpy's own fp32 power (each within an ulp of
    the correctly rounded value), and the exponent against a brute-force fraction."""
    for pairs, base in ((64, 1e6), (32, 10000.0), (16, 500000.0)):
        got = rope.laguna_inverse(pairs, base)
        torch_row = torch.pow(torch.tensor(base, dtype=torch.float32),
                              torch.arange(0, 2 * pairs, 2, dtype=torch.float32) / (2 * pairs)).numpy()
        numpy_row = np.power(np.float32(base), np.arange(0, 2 * pairs, 2, dtype=np.float32) / np.float32(2 * pairs))
        for other in (torch_row, numpy_row):
            gap = np.abs(got.view(np.int32).astype(np.int64) - other.astype(np.float32).view(np.int32))
            assert gap.max() <= 1
        assert got[0] == 1.0
        assert abs(float(got[-1]) / base ** ((2 * pairs - 2) / (2 * pairs)) - 1.0) < 2 ** -23


def test_laguna_angles_are_fp32_quotients():
    """theta equals numpy's own fp32 division (IEEE, correctly rounded), which pins the
    float64-then-round formation; column 0 (inverse 1) is the plain fp64 table's."""
    rows, pairs, base = 40960, 64, 1e6
    inverse = rope.laguna_inverse(pairs, base)
    cos, sin = rope.laguna_angle_table(rows, pairs, base)
    positions = np.arange(rows, dtype=np.float32)
    theta = positions[:, None] / inverse[None, :]
    assert theta.dtype == np.float32
    np.testing.assert_array_equal(cos, np.cos(theta.astype(np.float64)).astype(np.float32))
    np.testing.assert_array_equal(sin, np.sin(theta.astype(np.float64)).astype(np.float32))
    cos64, sin64 = rope.angle_table(rows, pairs, base)
    assert np.array_equal(cos[:, 0], cos64[:, 0]) and np.array_equal(sin[:, 0], sin64[:, 0])
    assert (cos[0] == 1.0).all() and (sin[0] == 0.0).all()
    # against numpy's float32 cos and sin, a different evaluation: within 2 fp32 ulps
    gap = np.abs(np.cos(theta).view(np.int32).astype(np.int64) - cos.view(np.int32))
    assert np.percentile(gap, 99.9) <= 2


def test_fp32_and_fp64_atlases_differ_by_the_angle_rounding():
    """The two arithmetics at the config's 40,960 x 64, base 1e6: they agree at small
    positions and part by up to half an fp32 ulp of theta (about 4e-3 rad near 40,960)."""
    cos32, sin32 = rope.laguna_angle_table(40960, 64, 1e6)
    cos64, sin64 = rope.angle_table(40960, 64, 1e6)
    dcos, dsin = np.abs(cos32 - cos64), np.abs(sin32 - sin64)
    print(f"max |dcos| {dcos.max():.3e} max |dsin| {dsin.max():.3e}; "
          f"rows < 4096: {dcos[:4096].max():.3e} {dsin[:4096].max():.3e}")
    assert 1e-3 < max(dcos.max(), dsin.max()) < 5e-3
    assert max(dcos[:256].max(), dsin[:256].max()) < 2e-5
    # the bound: half an ulp of the largest angle plus the inverse row's own rounding
    theta_max = 40959.0
    assert max(dcos.max(), dsin.max()) <= theta_max * 2.0 ** -24 * 2 + 1e-6

"""The device-built rotary angle atlas (csrc/rope_atlas.hip, kernels/qkv_rope/atlas.py).

Against the oracle's table (oracle/rope.py `angle_table`, the fp64 build of
tests/test_kernel_qk_norm_rope.py:51-66): bit-equal at the config's 40,960 x 64 for
theta = 1e6, and after growth on demand (models/laguna/layers/attention.py:235-243) with
the old rows kept. The attention step and the table-driven QK-norm + RoPE read an atlas
that grows past its last row and match the oracle there. A YaRN table (1 / freqs as the
frequencies) against the closed form. Both entry points, called directly, bit-equal to the
oracle for pair counts that leave lanes idle or span two runs of 64 pairs (the row past
the last untouched), at positions whose angles cross 2^25, where the kernels change from
their own Cody-Waite reduction to the device library's sincos.
"""

import numpy as np
import pytest
import torch

from mlx_omnia_amd.kernels.attention import AttentionStep, FixedKVCache, HipAttentionStep
from mlx_omnia_amd.kernels.qkv_rope import AngleAtlas, HipQkNormRope, QkvRope, rope_core
from mlx_omnia_amd.kernels.qkv_rope.atlas import rope_frequencies, rope_inverse_fp32
from mlx_omnia_amd.runtime import ops
from oracle import attention as attn
from oracle import rope
from oracle.bf16 import from_float
from util import assert_bf16_close, bits_of, to_device

pytestmark = pytest.mark.gpu


def test_config_table_bit_equal_to_oracle():
    print("atlas 40960 x 64 theta 1e6", flush=True)
    atlas = AngleAtlas(64, base=1e6, rows=40960, device="cuda")
    cos, sin = rope.angle_table(40960, 64, 1e6)
    got = atlas.atlas.cpu().numpy()
    assert got.shape == (40960, 128)
    assert np.array_equal(got[:, :64], cos) and np.array_equal(got[:, 64:], sin)


@pytest.mark.parametrize("pairs,first,rows", [(3, 0, 1000), (40, 33_554_000, 512),
                                             (100, 33_554_300, 300), (64, 10**9, 64)])
def test_entry_points_across_the_fast_reduction_limit(pairs, first, rows):
    print(f"atlas entry points pairs={pairs} first={first} rows={rows}", flush=True)
    width = 2 * pairs
    out = torch.full((rows + 1, width), 7.0, device="cuda")   # the last row must stay untouched
    freqs = torch.tensor(rope_frequencies(pairs, 1e4), dtype=torch.float64, device="cuda")
    ops.rope_angle_atlas(freqs, first, rows, out=out[:rows])
    cos, sin = rope.angle_table(rows, pairs, 1e4, first=first)
    got = out.cpu().numpy()
    assert np.array_equal(got[:rows, :pairs], cos) and np.array_equal(got[:rows, pairs:], sin)
    assert (got[rows] == 7.0).all()
    inverse = torch.tensor(rope_inverse_fp32(pairs, 1e4), dtype=torch.float32, device="cuda")
    ops.rope_angle_atlas_fp32(inverse, first, rows, out=out[:rows])
    cos, sin = rope.laguna_angle_table(rows, pairs, 1e4, first=first)
    got = out.cpu().numpy()
    assert np.array_equal(got[:rows, :pairs], cos) and np.array_equal(got[:rows, pairs:], sin)
    assert (got[rows] == 7.0).all()


def test_growth_keeps_old_rows_and_matches_oracle():
    atlas = AngleAtlas(32, base=10000.0, rows=100, device="cuda")
    first = atlas.atlas.clone()
    atlas.ensure(5000)
    assert atlas.rows >= 5001
    assert torch.equal(atlas.atlas[:100], first)
    cos, sin = rope.angle_table(atlas.rows, 32, 10000.0)
    got = atlas.atlas.cpu().numpy()
    assert np.array_equal(got[:, :32], cos) and np.array_equal(got[:, 32:], sin)
    rows = atlas(6000, 3)                        # the Angles contract grows too
    assert rows.shape == (3, 64) and atlas.rows >= 6003


def test_fp32_order_bit_equal_to_oracle_and_grows():
    """Laguna's fp32 op order (models/laguna/layers/attention.py:236-243) at the config's
    40,960 x 64, then grown past its last row (old rows kept), and a YaRN inverse row."""
    print("atlas fp32 order 40960 x 64 theta 1e6", flush=True)
    atlas = AngleAtlas(64, base=1e6, rows=40960, device="cuda", arithmetic="fp32")
    cos, sin = rope.laguna_angle_table(40960, 64, 1e6)
    got = atlas.atlas.cpu().numpy()
    assert np.array_equal(got[:, :64], cos) and np.array_equal(got[:, 64:], sin)
    kept = atlas.atlas.clone()
    atlas.ensure(70000)
    assert torch.equal(atlas.atlas[:40960], kept)
    cos, sin = rope.laguna_angle_table(atlas.rows, 64, 1e6)
    got = atlas.atlas.cpu().numpy()
    assert np.array_equal(got[:, :64], cos) and np.array_equal(got[:, 64:], sin)
    freqs = (1e4 ** (np.arange(0, 64, 2) / 64) * np.linspace(1.0, 8.0, 32)).astype(np.float32)
    yarn = AngleAtlas(32, inverse_frequencies=freqs, rows=4096, device="cuda", arithmetic="fp32")
    cos, sin = rope.laguna_angle_table(4096, 32, inverse=freqs)
    got = yarn.atlas.cpu().numpy()
    assert np.array_equal(got[:, :32], cos) and np.array_equal(got[:, 32:], sin)


def test_yarn_frequencies():
    pairs = 32
    freqs = 1e4 ** (np.arange(0, 2 * pairs, 2) / (2 * pairs)) * np.linspace(1.0, 8.0, pairs)
    atlas = AngleAtlas(pairs, inverse_frequencies=freqs, rows=2048, device="cuda")
    theta = np.arange(2048)[:, None] * (1.0 / freqs)[None, :]
    got = atlas.atlas.cpu().numpy()
    ulp = np.spacing(np.float32(1.0))
    assert np.abs(got[:, :pairs] - np.cos(theta)).max() <= ulp
    assert np.abs(got[:, pairs:] - np.sin(theta)).max() <= ulp


def test_attention_step_grows_the_atlas_past_its_last_row():
    heads, kv_heads, capacity, pairs = 8, 2, 256, 64
    rng = np.random.default_rng(31)
    qw, kw = (from_float(1 + 0.1 * rng.standard_normal(128)) for _ in range(2))
    cache = FixedKVCache.empty(kv_heads, capacity, 128, device="cuda")
    atlas = AngleAtlas(pairs, base=1e6, rows=16, device="cuda")
    step = AttentionStep(cache, heads=heads, kv_heads=kv_heads, head_dim=128, scale=128 ** -0.5,
                         dtype=torch.bfloat16, query_weight=to_device(qw), key_weight=to_device(kw),
                         eps=1e-6, rotary_pairs=pairs, angles=atlas)
    assert isinstance(step.strategy, HipAttentionStep)
    keys = np.zeros((kv_heads, capacity, 128), np.uint16)
    values = keys.copy()
    cos, sin = rope.angle_table(64, pairs, 1e6)
    for position in range(40):
        q = from_float(rng.standard_normal(heads * 128))
        k = from_float(rng.standard_normal(kv_heads * 128))
        v = from_float(rng.standard_normal(kv_heads * 128))
        out = step(*(to_device(t).reshape(1, 1, -1) for t in (q, k, v)))
        row = np.concatenate([cos[position], sin[position]])
        want, keys, values = attn.decode_step(q, k, v, qw, kw, row, keys, values, position,
                                              window=0, scale=128 ** -0.5, eps=1e-6, pairs=pairs)
        assert_bf16_close(bits_of(out.reshape(heads, 128)), want, min_exact=0.99)
    assert atlas.rows >= 40


def test_qk_norm_rope_reads_a_growing_atlas():
    heads, kv_heads, d, pairs, t = 4, 2, 128, 64, 8
    rng = np.random.default_rng(32)
    qw, kw = (from_float(1 + 0.1 * rng.standard_normal(d)) for _ in range(2))
    atlas = AngleAtlas(pairs, base=1e6, rows=64, device="cuda")
    facade = QkvRope(lambda x: x, heads=heads, kv_heads=kv_heads, head_dim=d,
                     rope=lambda x, o: rope_core(x, o, base=1e6), eps=1e-6,
                     q_norm=to_device(qw), k_norm=to_device(kw), angles=atlas, rotary_pairs=pairs)
    assert isinstance(facade.strategy, HipQkNormRope)
    fused = from_float(rng.standard_normal((1, t, (heads + 2 * kv_heads) * d)))
    offset = 3000
    q, k, _ = facade(to_device(fused), offset)
    assert atlas.rows >= offset + t
    cos, sin = rope.angle_table(offset + t, pairs, 1e6)
    raw = fused[0]
    want_q, want_k = rope.qk_norm_rope(
        raw[:, : heads * d].reshape(t, heads, d), raw[:, heads * d : (heads + kv_heads) * d].reshape(t, kv_heads, d),
        qw, kw, cos, sin, offset, 1e-6, pairs)
    assert_bf16_close(bits_of(q[0]), want_q)
    assert_bf16_close(bits_of(k[0]), want_k)

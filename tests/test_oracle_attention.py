"""The decode-attention oracle (oracle/attention.py) pinned without its own formula.

- attention: torch's scaled_dot_product_attention in float64 over the same rows (with
  the kv heads repeated for grouped queries); closed forms: one attended row returns its
  value row exactly, equal keys return the mean of the values, one dominant key returns
  its value row; rows past the attended count never enter (NaN there changes nothing);
- the cache geometry: the fixed cache and the ring's write rows and counts against
  core/cache/kv.py's definitions, including the wrap;
- the new rows: the key written is oracle.rope.norm_rotate's (pinned in
  test_oracle_rope.py), the value row is written verbatim, other rows are untouched;
- planted mistakes (kv head h % kv_heads, no scale, the key left unrotated) fail.
"""

import numpy as np
import pytest
import torch

from oracle import attention as attn
from oracle.bf16 import from_float, to_f32, ulp_distance
from oracle.rope import angle_table

D = 128


def _angle_row(position, pairs, base=10000.0):
    cos, sin = angle_table(1, pairs, base, first=position)
    return np.concatenate([cos[0], sin[0]]).astype(np.float32)


def _setup(rng, heads=8, kv_heads=2, capacity=64):
    raw_q = from_float(rng.standard_normal(heads * D))
    raw_k = from_float(rng.standard_normal(kv_heads * D))
    raw_v = from_float(rng.standard_normal(kv_heads * D))
    qw = from_float(1 + 0.1 * rng.standard_normal(D))
    kw = from_float(1 + 0.1 * rng.standard_normal(D))
    kc = from_float(rng.standard_normal((kv_heads, capacity, D)))
    vc = from_float(rng.standard_normal((kv_heads, capacity, D)))
    return raw_q, raw_k, raw_v, qw, kw, kc, vc


def test_attend_matches_torch_sdpa_float64():
    rng = np.random.default_rng(0)
    heads, kv_heads, rows = 8, 2, 37
    q = from_float(rng.standard_normal((heads, D)))
    k = from_float(rng.standard_normal((kv_heads, rows, D)))
    v = from_float(rng.standard_normal((kv_heads, rows, D)))
    scale = D ** -0.5
    got = attn.attend(q, k, v, scale)
    tq = torch.from_numpy(to_f32(q)).double()[None, :, None, :]
    tk = torch.from_numpy(to_f32(k)).double().repeat_interleave(heads // kv_heads, dim=0)[None]
    tv = torch.from_numpy(to_f32(v)).double().repeat_interleave(heads // kv_heads, dim=0)[None]
    want = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, scale=scale)[0, :, 0]
    assert ulp_distance(got, from_float(want.float().numpy())).max() <= 1


def test_attend_closed_forms():
    rng = np.random.default_rng(1)
    q = from_float(rng.standard_normal((2, D)))
    v = from_float(rng.standard_normal((1, 5, D)))
    one = attn.attend(q, from_float(rng.standard_normal((1, 1, D))), v[:, :1], 0.1)
    assert np.array_equal(one, np.repeat(v[:, 0], 2, axis=0))            # one row: its value
    same = np.repeat(from_float(rng.standard_normal((1, 1, D))), 5, axis=1)
    mean = to_f32(v)[0].astype(np.float64).mean(axis=0)
    got = attn.attend(q, same, v, 0.1)
    # equal keys: the mean of the values (p = 1/5 is inexact, so near-zero means may land
    # on either side of a tiny value: compare at bf16 resolution)
    assert np.allclose(to_f32(got[0]), mean, rtol=2.0**-8, atol=1e-6)
    dominant = from_float(rng.standard_normal((1, 5, D)) * 0.01)
    dominant[0, 3] = from_float(40 * to_f32(q[0]))
    got = attn.attend(q[:1], dominant, v, 1.0)
    assert np.array_equal(got[0], v[0, 3])                              # one key dominates


def test_step_rows_fixed_and_ring():
    assert attn.step_rows(0, 64, 0) == (0, 1)
    assert attn.step_rows(63, 64, 0) == (63, 64)
    assert attn.step_rows(5, 64, 64) == (5, 6)
    assert attn.step_rows(64, 64, 64) == (0, 64)       # the ring wraps: slot 0, all filled
    assert attn.step_rows(130, 64, 64) == (2, 64)


@pytest.mark.parametrize("window", [0, 64])
def test_decode_step_writes_the_new_row_and_ignores_rows_past_the_count(window):
    rng = np.random.default_rng(2)
    raw_q, raw_k, raw_v, qw, kw, kc, vc = _setup(rng)
    position = 70 if window else 20
    row = _angle_row(position, 64)
    out, keys, values = attn.decode_step(raw_q, raw_k, raw_v, qw, kw, row, kc, vc, position,
                                         window=window, scale=D ** -0.5, eps=1e-6, pairs=64)
    write, count = attn.step_rows(position, 64, window)
    assert np.array_equal(keys[:, write], attn.roped(raw_k, kw, row, 1e-6, 64, 1.0))
    assert np.array_equal(values[:, write], raw_v.reshape(2, D))
    untouched = [r for r in range(64) if r != write]
    assert np.array_equal(keys[:, untouched], kc[:, untouched])
    if count < 64:
        poisoned_k, poisoned_v = kc.copy(), vc.copy()
        poisoned_k[:, count:] = 0x7FC0  # NaN
        poisoned_v[:, count:] = 0x7FC0
        again, _, _ = attn.decode_step(raw_q, raw_k, raw_v, qw, kw, row, poisoned_k, poisoned_v,
                                       position, window=window, scale=D ** -0.5, eps=1e-6, pairs=64)
        assert np.array_equal(out, again)


@pytest.mark.parametrize("kind", ["kv_head_modulo", "no_scale", "key_unrotated"])
def test_planted_mistakes_fail(kind):
    rng = np.random.default_rng(3)
    raw_q, raw_k, raw_v, qw, kw, kc, vc = _setup(rng)
    row = _angle_row(30, 64)
    scale = D ** -0.5
    good, keys, values = attn.decode_step(raw_q, raw_k, raw_v, qw, kw, row, kc, vc, 30,
                                          window=0, scale=scale, eps=1e-6, pairs=64)
    q = attn.roped(raw_q, qw, row, 1e-6, 64, 1.0)
    if kind == "kv_head_modulo":
        swapped = keys[[0, 1] * 4][:, :31].reshape(8, 1, 31, D)
        vals = values[[0, 1] * 4][:, :31].reshape(8, 1, 31, D)
        bad = np.stack([attn.attend(q[h:h + 1], swapped[h], vals[h], scale)[0] for h in range(8)])
    elif kind == "no_scale":
        bad = attn.attend(q, keys[:, :31], values[:, :31], 1.0)
    else:
        plain = keys.copy()
        plain[:, 30] = raw_k.reshape(2, D)
        bad = attn.attend(q, plain[:, :31], values[:, :31], scale)
    assert not np.array_equal(good, bad)

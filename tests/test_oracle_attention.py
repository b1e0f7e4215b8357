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


# ---- sink_attend: the attention of a layer with learned sink logits --------------------
#
# Pinned against a formula of its own: torch float64 softmax over the scores with the
# sink prepended as one more column, that column dropped, the rest times the values
# (what mx.fast.scaled_dot_product_attention(sinks=...) computes, the reference's own
# parity target, tests/test_kernel_sink_attention.py:118-132). Closed forms: no attended
# row gives zeros; a sink far below the scores gives the plain softmax. Mistakes the
# comparison catches: the sink left out, the mask left out, the scale applied to the
# mask, kv head h % kv_heads.

def _sink_case(seed, heads=8, kv_heads=2, rows=40, head_dim=64):
    rng = np.random.default_rng(seed)
    q = from_float(rng.standard_normal((heads, head_dim)))
    k = from_float(rng.standard_normal((kv_heads, rows, head_dim)))
    v = from_float(rng.standard_normal((kv_heads, rows, head_dim)))
    sinks = from_float(2.0 * rng.standard_normal(heads))
    return q, k, v, sinks


def _torch_sink(q, k, v, sinks, mask, scale, *, drop_sink=False, drop_mask=False, scale_mask=False,
                modulo=False):
    heads, kv_heads, rows = q.shape[0], k.shape[0], k.shape[1]
    gqa = heads // kv_heads
    qt = torch.from_numpy(to_f32(q)).double()
    kt = torch.from_numpy(to_f32(k)).double()
    vt = torch.from_numpy(to_f32(v)).double()
    st = torch.from_numpy(to_f32(sinks)).double()
    if mask is None:
        additive = torch.zeros(rows, dtype=torch.float64)
    elif mask.dtype == np.bool_:
        additive = torch.where(torch.from_numpy(mask), 0.0, float("-inf")).double()
    else:
        additive = torch.from_numpy(np.asarray(mask, dtype=np.float64))
    if drop_mask:
        additive = torch.zeros(rows, dtype=torch.float64)
    out = []
    for h in range(heads):
        kvh = h % kv_heads if modulo else h // gqa
        dots = kt[kvh] @ qt[h]
        scores = (dots + additive) * scale if scale_mask else dots * scale + additive
        if drop_sink:
            probs = torch.softmax(scores, dim=0)
        else:
            probs = torch.softmax(torch.cat([st[h : h + 1], scores]), dim=0)[1:]
        out.append(probs @ vt[kvh])
    return torch.stack(out).numpy()


def _band(rows, window):
    return np.arange(rows) >= rows - window


@pytest.mark.parametrize("mask_kind", ["none", "band", "additive"])
def test_sink_attend_matches_torch_float64(mask_kind):
    q, k, v, sinks = _sink_case(1)
    rows = k.shape[1]
    mask = {"none": None, "band": _band(rows, 16),
            "additive": np.where(np.arange(rows) % 7 == 3, -np.inf, 0.25 * np.sin(np.arange(rows)))}[mask_kind]
    got = attn.sink_attend(q, k, v, sinks, mask, 0.125)
    want = _torch_sink(q, k, v, sinks, mask, 0.125)
    assert np.abs(to_f32(got) - want).max() <= 2.0 ** -8 * np.abs(want).max()
    assert np.mean(ulp_distance(got, from_float(want.astype(np.float32))) == 0) >= 0.99


def test_sink_attend_closed_forms():
    q, k, v, sinks = _sink_case(2)
    rows = k.shape[1]
    none = attn.sink_attend(q, k, v, sinks, np.zeros(rows, bool), 0.125)
    assert not to_f32(none).any()
    empty = attn.sink_attend(q, k[:, :0], v[:, :0], sinks, None, 0.125)
    assert empty.shape == q.shape and not to_f32(empty).any()
    low = from_float(np.full(q.shape[0], -1e30))
    plain = attn.sink_attend(q, k, v, low, None, 0.125)
    want = _torch_sink(q, k, v, low, None, 0.125, drop_sink=True)
    assert np.abs(to_f32(plain) - want).max() <= 2.0 ** -8 * np.abs(want).max()


@pytest.mark.parametrize("mistake", ["drop_sink", "drop_mask", "scale_mask", "modulo"])
def test_sink_attend_comparison_tells_mistakes_apart(mistake):
    q, k, v, sinks = _sink_case(3)
    rows = k.shape[1]
    mask = np.where(np.arange(rows) % 5 == 0, -np.inf, 0.5 * np.cos(np.arange(rows)))
    got = to_f32(attn.sink_attend(q, k, v, sinks, mask, 0.125))
    wrong = _torch_sink(q, k, v, sinks, mask, 0.125, **{mistake: True})
    assert np.abs(got - wrong).max() > 4 * 2.0 ** -8 * np.abs(wrong).max()

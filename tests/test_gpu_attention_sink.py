"""The sink-logit attention (`omnia_attention_sink_decode`, csrc/attention_sink.hip) against
the oracle (oracle/attention.py `sink_attend`), and the step that binds it.

Mirrors the reference's `sink_attention` and `SinkAttentionStep`
(core/kernels/attention/sink.py) and its test's shapes (tests/test_kernel_sink_attention.py:
gpt-oss geometry, 64 query heads over 8 kv heads, head_dim 64, 129, 600 and 1031 cached
rows, the sliding band of 128 and the full layer), plus 32,768 rows, grouped queries 1, 2
and 4, an empty cache, a buffer wider than its rows, an additive mask with finite values,
and a mask that hides every row.

Bar: the north-star bf16 bar (assert_bf16_close) with at least 99% of the outputs
bit-identical.
"""

import numpy as np
import pytest
import torch

from mlx_omnia_amd.runtime import ops
from oracle import attention as attn
from oracle.bf16 import from_float
from util import assert_bf16_close, bits_of, to_device

pytestmark = pytest.mark.gpu


def _case(seed, heads, kv_heads, rows, capacity=None):
    rng = np.random.default_rng(seed)
    capacity = capacity or rows
    q = from_float(rng.standard_normal((heads, 64)))
    k = from_float(rng.standard_normal((kv_heads, capacity, 64)))
    v = from_float(rng.standard_normal((kv_heads, capacity, 64)))
    sinks = from_float(2.0 * rng.standard_normal(heads))
    return q, k, v, sinks


def _run(q, k, v, sinks, rows, mask, scale=0.125):
    kd, vd = to_device(k)[None], to_device(v)[None]
    got = ops.attention_sink_decode(to_device(q), kd[:, :, :rows], vd[:, :, :rows], to_device(sinks),
                                    None if mask is None else torch.from_numpy(mask).cuda(), scale)
    want = attn.sink_attend(q, k[:, :rows], v[:, :rows], sinks, mask, scale)
    return bits_of(got), want


@pytest.mark.parametrize("rows", [129, 600, 1031, 32768])
@pytest.mark.parametrize("sliding", [False, True])
def test_matches_oracle_at_gpt_oss_geometry(rows, sliding):
    print(f"attention_sink_decode rows={rows} sliding={sliding}", flush=True)
    q, k, v, sinks = _case(rows + sliding, 64, 8, rows)
    mask = (np.arange(rows) >= rows - 128) if sliding else None
    got, want = _run(q, k, v, sinks, rows, mask)
    assert_bf16_close(got, want, min_exact=0.99)


@pytest.mark.parametrize("heads,kv_heads,rows,capacity", [(4, 4, 300, 512), (8, 4, 1, 256), (16, 4, 2047, 2304),
                                                          (8, 1, 5000, 5000)])
def test_grouped_queries_and_wide_buffers(heads, kv_heads, rows, capacity):
    print(f"attention_sink_decode heads={heads} kv_heads={kv_heads} rows={rows}", flush=True)
    q, k, v, sinks = _case(heads * rows, heads, kv_heads, rows, capacity)
    got, want = _run(q, k, v, sinks, rows, None)
    assert_bf16_close(got, want, min_exact=0.99)


def test_additive_mask_empty_cache_and_every_row_masked():
    q, k, v, sinks = _case(5, 16, 2, 700)
    mask = np.where(np.arange(700) % 9 == 4, -np.inf, 0.3 * np.sin(np.arange(700))).astype(np.float32)
    got, want = _run(q, k, v, sinks, 700, mask)
    assert_bf16_close(got, want, min_exact=0.99)
    hidden, _ = _run(q, k, v, sinks, 700, np.zeros(700, bool))
    assert not np.any(hidden & 0x7FFF)
    empty, _ = _run(q, k, v, sinks, 0, None)
    assert not np.any(empty & 0x7FFF)


def test_step_binds_the_sink_kernel_and_matches_the_core_chain():
    from mlx_omnia_amd.kernels.attention import AttentionStep, HipSinkAttentionStep, KVCache
    from mlx_omnia_amd.kernels.qkv_rope.atlas import AngleAtlas

    rng = np.random.default_rng(6)
    heads, kv_heads = 64, 8
    sinks = torch.from_numpy(2.0 * rng.standard_normal(heads)).to(torch.bfloat16).cuda()
    atlas = AngleAtlas(32, base=150000.0, device="cuda")
    declare = dict(heads=heads, kv_heads=kv_heads, head_dim=64, scale=0.125, dtype=torch.bfloat16,
                   rotary_pairs=32, angles=atlas, sinks=sinks)
    ours, core = KVCache(), KVCache()
    step = AttentionStep(ours, **declare)
    reference = AttentionStep(core, reference=True, **declare)
    assert isinstance(step.strategy, HipSinkAttentionStep)

    def raw(t, count):
        return torch.from_numpy(rng.standard_normal((1, t, count * 64))).to(torch.bfloat16).cuda()

    prefill = [raw(300, heads), raw(300, kv_heads), raw(300, kv_heads)]
    step(*prefill, mask="causal")
    reference(*prefill, mask="causal")
    for i in range(3):
        inputs = [raw(1, heads), raw(1, kv_heads), raw(1, kv_heads)]
        band = torch.arange(ours.offset + 1, device="cuda") >= ours.offset + 1 - 128 if i == 2 else None
        got = step(*inputs, mask=band)
        want = reference(*inputs, mask=band)
        assert got.shape == (1, heads, 1, 64)
        assert_bf16_close(bits_of(got.reshape(heads, 64)), bits_of(want.reshape(heads, 64)), min_exact=0.98)
    assert ours.offset == core.offset == 303

"""HIP QK-norm + RoPE (table and epilogue) against the CPU oracle.

Bar: within 2 bf16 ulp and atol/rtol 1e-2 of the oracle; in practice the kernel is
bit-exact except where the fp32 summation order of a head's sum of squares moves a
rounding. Cases: the configs (T=64 decode rows, T=4096 prefill; q [T,32,128], k
[T,8,128], cos/sin [40960,64] for theta=1e6, offset uniform in [0, 32768)), the
reference test's shapes (12/4 heads, partial rotary, the YaRN mscale), head_dim 64 and
256, the last table row, q/k read in place from fused qkv rows, the reference's
cos||sin atlas layout, empty and single-token segments.
"""

import math

import numpy as np
import pytest
import torch

from mlx_omnia_amd.kernels.qkv_rope import AngleTable, HipQkNormRope, HipRopeEpilogue, QkvRope, rope_core
from mlx_omnia_amd.runtime import ops
from oracle import rope
from oracle.add_norm import rms_norm
from oracle.bf16 import from_float
from util import assert_bf16_close, bits_of, exact_fraction, f32_to_device, to_device

pytestmark = pytest.mark.gpu

EPS = 1e-6
MSCALE = 1.3465735912322998
TABLE_ROWS = 40960
_TABLES = {}


def _table(pairs, base=1e6, rows=TABLE_ROWS):
    key = (pairs, base, rows)
    if key not in _TABLES:
        _TABLES[key] = rope.angle_table(rows, pairs, base)
    return _TABLES[key]


def _inputs(length, hq, hkv, d, seed):
    rng = np.random.default_rng(seed)
    return (
        from_float(rng.standard_normal((length, hq, d))),
        from_float(rng.standard_normal((length, hkv, d))),
        from_float(1.0 + 0.1 * rng.standard_normal(d)),
        from_float(1.0 + 0.1 * rng.standard_normal(d)),
    )


CASES = [
    # length, q heads, kv heads, head_dim, rotary pairs, offset, mscale, table layout
    (64, 32, 8, 128, 64, 21_537, 1.0, "separate"),
    (4096, 32, 8, 128, 64, 28_301, 1.0, "separate"),
    (5, 12, 4, 128, 32, 3, MSCALE, "atlas"),
    (5, 12, 4, 128, 64, 3, MSCALE, "atlas"),
    (5, 12, 4, 64, 16, 3, MSCALE, "atlas"),
    (7, 8, 2, 256, 128, 100, 1.0, "separate"),
    (3, 8, 2, 256, 64, 9, 1.0, "separate"),
    (6, 16, 4, 64, 32, 77, 1.0, "separate"),        # full rotary, 4 lanes per head
    (4, 20, 4, 64, 32, 5, MSCALE, "atlas"),         # ... head counts not a multiple of 16
    (9, 6, 2, 256, 128, 31_000, MSCALE, "atlas"),   # full rotary, 16 lanes per head, scaled
    (1, 32, 8, 128, 64, TABLE_ROWS - 1, 1.0, "separate"),
    (0, 32, 8, 128, 64, 0, 1.0, "separate"),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"T{c[0]}-{c[1]}x{c[2]}-D{c[3]}-P{c[4]}-{c[7]}")
def test_table_kernel_matches_oracle(case):
    length, hq, hkv, d, pairs, offset, mscale, layout = case
    print(f"qk_norm_rope {case}", flush=True)
    raw_q, raw_k, qw, kw = _inputs(length, hq, hkv, d, seed=length + d + pairs)
    cos, sin = _table(pairs)
    if layout == "atlas":
        atlas = f32_to_device(np.concatenate([cos[: offset + length + 1], sin[: offset + length + 1]], -1))
        cos_t, sin_t = atlas[:, :pairs], atlas[:, pairs:]
    else:
        cos_t, sin_t = f32_to_device(cos), f32_to_device(sin)
    q, k = ops.qk_norm_rope(
        to_device(raw_q), to_device(raw_k), to_device(qw), to_device(kw), cos_t, sin_t,
        offset=offset, eps=EPS, rotary_pairs=pairs, mscale=mscale,
    )
    torch.cuda.synchronize()
    want_q, want_k = rope.qk_norm_rope(raw_q, raw_k, qw, kw, cos, sin, offset, EPS, pairs, mscale)
    assert q.shape == (hq, length, d) and k.shape == (hkv, length, d)
    assert_bf16_close(bits_of(q), want_q)
    assert_bf16_close(bits_of(k), want_k)
    assert exact_fraction(bits_of(q), want_q) > 0.99


def test_position_zero_identity_and_tail_through_kernel():
    raw_q, raw_k, qw, kw = _inputs(4, 12, 4, 128, seed=2)
    cos, sin = _table(32)
    q, k = ops.qk_norm_rope(
        to_device(raw_q), to_device(raw_k), to_device(qw), to_device(kw),
        f32_to_device(cos[:8]), f32_to_device(sin[:8]), offset=0, eps=EPS, rotary_pairs=32,
    )
    normed_q = rms_norm(raw_q, qw, EPS).transpose(1, 0, 2)
    got = bits_of(q)
    assert np.array_equal(got[:, 0], normed_q[:, 0])             # position 0: identity
    assert_bf16_close(got[..., 64:], normed_q[..., 64:], max_ulp=0)  # tail: the norm


def test_reads_q_and_k_in_place_from_fused_rows_via_facade():
    hq, hkv, d, length, offset = 16, 4, 128, 33, 500
    rng = np.random.default_rng(9)
    fused = from_float(rng.standard_normal((1, length, (hq + 2 * hkv) * d)))
    qw, kw = from_float(1 + 0.1 * rng.standard_normal(d)), from_float(1 + 0.1 * rng.standard_normal(d))
    cos, sin = _table(64, rows=1024)
    table = AngleTable(f32_to_device(cos), f32_to_device(sin))
    prologue = QkvRope(lambda x: x, heads=hq, kv_heads=hkv, head_dim=d,
                       rope=lambda x, o: rope_core(x, o, base=1e6), eps=EPS,
                       q_norm=to_device(qw), k_norm=to_device(kw), angles=table, rotary_pairs=64)
    assert isinstance(prologue.strategy, HipQkNormRope)
    q, k, v = prologue(to_device(fused), offset)
    assert q.shape == (1, hq, length, d) and k.shape == (1, hkv, length, d) and v.shape == (1, hkv, length, d)
    raw = fused[0]
    want_q, want_k = rope.qk_norm_rope(
        raw[:, : hq * d].reshape(length, hq, d), raw[:, hq * d : (hq + hkv) * d].reshape(length, hkv, d),
        qw, kw, cos, sin, offset, EPS, 64,
    )
    assert_bf16_close(bits_of(q[0]), want_q)
    assert_bf16_close(bits_of(k[0]), want_k)
    want_v = raw[:, (hq + hkv) * d :].reshape(length, hkv, d).transpose(1, 0, 2)
    assert np.array_equal(bits_of(v[0]), want_v)


EPILOGUE = [(1, 0), (1, 4095), (64, 137), (4096, 28_301), (3, 32_767), (200, 16_777_000), (512, 9_000_000)]


@pytest.mark.parametrize("length,offset", EPILOGUE)
def test_epilogue_matches_oracle(length, offset):
    print(f"rope_epilogue T={length} offset={offset}", flush=True)
    hq, hkv, d = 32, 8, 128
    rng = np.random.default_rng(length + offset)
    fused = from_float(rng.standard_normal((length, (hq + 2 * hkv) * d)))
    qw, kw = from_float(1 + 0.1 * rng.standard_normal(d)), from_float(1 + 0.1 * rng.standard_normal(d))
    q, k = ops.rope_epilogue(
        to_device(fused), to_device(qw), to_device(kw), query_heads=hq, kv_heads=hkv,
        head_dim=d, offset=offset, log2_base=math.log2(1e6), eps=EPS,
    )
    torch.cuda.synchronize()
    want_q, want_k = rope.rope_epilogue(fused, hq, hkv, d, qw, kw, offset, 1e6, EPS)
    assert_bf16_close(bits_of(q), want_q)
    assert_bf16_close(bits_of(k), want_k)
    assert exact_fraction(bits_of(q), want_q) > 0.99


@pytest.mark.parametrize("head_dim,hq,hkv,length,offset", [(64, 20, 4, 33, 901), (256, 8, 2, 17, 12_345)])
def test_epilogue_other_head_dims(head_dim, hq, hkv, length, offset):
    print(f"rope_epilogue D={head_dim} hq={hq} hkv={hkv} T={length}", flush=True)
    rng = np.random.default_rng(head_dim + length)
    fused = from_float(rng.standard_normal((length, (hq + 2 * hkv) * head_dim)))
    qw = from_float(1 + 0.1 * rng.standard_normal(head_dim))
    kw = from_float(1 + 0.1 * rng.standard_normal(head_dim))
    q, k = ops.rope_epilogue(
        to_device(fused), to_device(qw), to_device(kw), query_heads=hq, kv_heads=hkv,
        head_dim=head_dim, offset=offset, log2_base=math.log2(1e6), eps=EPS,
    )
    torch.cuda.synchronize()
    want_q, want_k = rope.rope_epilogue(fused, hq, hkv, head_dim, qw, kw, offset, 1e6, EPS)
    assert_bf16_close(bits_of(q), want_q)
    assert_bf16_close(bits_of(k), want_k)


def test_epilogue_facade_resolution_and_segment():
    hq, hkv, d = 32, 4, 128
    rng = np.random.default_rng(5)
    fused = from_float(rng.standard_normal((1, 9, (hq + 2 * hkv) * d)))
    qw, kw = from_float(1 + 0.1 * rng.standard_normal(d)), from_float(1 + 0.1 * rng.standard_normal(d))
    prologue = QkvRope(lambda x: x, heads=hq, kv_heads=hkv, head_dim=d,
                       rope=lambda x, o: rope_core(x, o, base=1e6), eps=EPS,
                       q_norm=to_device(qw), k_norm=to_device(kw), base=1e6)
    assert isinstance(prologue.strategy, HipRopeEpilogue)
    q, k, v = prologue(to_device(fused), 77)
    want_q, want_k = rope.rope_epilogue(fused[0], hq, hkv, d, qw, kw, 77, 1e6, EPS)
    assert_bf16_close(bits_of(q[0]), want_q)
    assert_bf16_close(bits_of(k[0]), want_k)


def test_golden_fixture():
    golden = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "qk_norm_rope.npz")
    q, k = ops.qk_norm_rope(
        to_device(golden["raw_q"]), to_device(golden["raw_k"]), to_device(golden["q_weight"]),
        to_device(golden["k_weight"]), f32_to_device(golden["cos"]), f32_to_device(golden["sin"]),
        offset=int(golden["offset"]), eps=float(golden["eps"]),
        rotary_pairs=int(golden["pairs"]), mscale=float(golden["mscale"]),
    )
    assert_bf16_close(bits_of(q), golden["q"])
    assert_bf16_close(bits_of(k), golden["k"])
    qe, ke = ops.rope_epilogue(
        to_device(golden["fused"]), to_device(golden["q_weight"]), to_device(golden["k_weight"]),
        query_heads=int(golden["hq"]), kv_heads=int(golden["hkv"]), head_dim=128,
        offset=int(golden["epilogue_offset"]), log2_base=math.log2(1e6), eps=float(golden["eps"]),
    )
    assert_bf16_close(bits_of(qe), golden["epilogue_q"])
    assert_bf16_close(bits_of(ke), golden["epilogue_k"])

"""HIP MXFP4 routed-expert kernels (csrc/moe_mxfp4.hip) against the oracle
(oracle/mxfp4.py).

Mirrors the reference's mxfp4 strategies (core/kernels/gate_up/mxfp4.py,
core/kernels/down_combine/mxfp4.py): the interleaved layout, the projection bias, the
clamped swiglu_oai. Shapes: gpt-oss-120b's routed MLP (hidden and inner 2880, 128
experts, top-4: 90 groups per row, not a multiple of the 64 lanes) and a small one;
the clamp off and biting; no bias; invalid expert ids; no residual; 1 and 16 slots.

The kernels decode with gfx950's v_cvt_scalef32_pk_bf16_fp4 and sum in fp32 in their own
order; the oracle rounds the exact dot product plus bias once. Bar: the north-star bf16
bar (assert_bf16_close) with at least 99% of the outputs bit-identical.
"""

import numpy as np
import pytest
import torch

from mlx_omnia_amd.runtime import ops
from oracle import mxfp4
from oracle.bf16 import from_float, to_f32
from util import assert_bf16_close, bits_of, f32_to_device, to_device

pytestmark = pytest.mark.gpu

HIDDEN, INNER, EXPERTS = 1024, 512, 8


def _leaf(rng, experts, rows, features, bias=True):
    """(oracle Stack, device Mxfp4Leaf): random codes, group scales near 2^-7, a bias."""
    words = rng.integers(0, 1 << 32, size=(experts, rows, features // 8), dtype=np.uint64).astype(np.uint32)
    scales = rng.integers(119, 123, size=(experts, rows, features // 32)).astype(np.uint8)
    b = from_float(0.25 * rng.standard_normal((experts, rows))) if bias else None
    stack = mxfp4.Stack(words, scales, b)
    leaf = ops.Mxfp4Leaf(torch.from_numpy(words.view(np.int32)).cuda(), torch.from_numpy(scales).cuda(),
                         to_device(b) if bias else None)
    return stack, leaf


def _ids(values):
    return torch.tensor(values, dtype=torch.int32, device="cuda")


@pytest.mark.parametrize("limit", [7.0, 0.5, None])
def test_gate_up_matches_oracle(limit):
    print(f"moe_gate_up_mxfp4 limit={limit}", flush=True)
    rng = np.random.default_rng(1 if limit is None else int(limit * 10))
    stack, leaf = _leaf(rng, EXPERTS, 2 * INNER, HIDDEN)
    x = from_float(2 * rng.standard_normal(HIDDEN))
    chosen = [5, 0, 7, 2]
    got = ops.moe_gate_up_mxfp4(to_device(x), leaf, _ids(chosen), limit=limit)
    assert_bf16_close(bits_of(got), mxfp4.gate_up(x, stack, chosen, limit), min_exact=0.99)


def test_gate_up_gpt_oss_shape_and_no_bias():
    print("moe_gate_up_mxfp4 gpt-oss-120b", flush=True)
    rng = np.random.default_rng(2)
    stack, leaf = _leaf(rng, 128, 2 * 2880, 2880)
    x = from_float(rng.standard_normal(2880))
    chosen = [17, 127, 64, 3]
    got = ops.moe_gate_up_mxfp4(to_device(x), leaf, _ids(chosen), limit=7.0)
    assert_bf16_close(bits_of(got), mxfp4.gate_up(x, stack, chosen, 7.0), min_exact=0.99)
    bare_stack, bare = _leaf(rng, EXPERTS, 2 * INNER, HIDDEN, bias=False)
    x = from_float(rng.standard_normal(HIDDEN))
    got = ops.moe_gate_up_mxfp4(to_device(x), bare, _ids([1, 4]), limit=7.0)
    assert_bf16_close(bits_of(got), mxfp4.gate_up(x, bare_stack, [1, 4], 7.0), min_exact=0.99)


def test_gate_up_invalid_ids_give_zeros():
    rng = np.random.default_rng(3)
    stack, leaf = _leaf(rng, EXPERTS, 2 * INNER, HIDDEN)
    x = from_float(rng.standard_normal(HIDDEN))
    got = bits_of(ops.moe_gate_up_mxfp4(to_device(x), leaf, _ids([-1, 3, EXPERTS]), limit=7.0))
    assert np.all(got[0] == 0) and np.all(got[2] == 0)
    assert_bf16_close(got[1:2], mxfp4.gate_up(x, stack, [3], 7.0), min_exact=0.99)


def _down(rng, slots, hidden=HIDDEN, inner=INNER, experts=EXPERTS, bias=True):
    stack, leaf = _leaf(rng, experts, hidden, inner, bias)
    act = from_float(rng.standard_normal((slots, inner)))
    weights = rng.dirichlet(np.ones(slots)).astype(np.float32)
    residual = from_float(rng.standard_normal(hidden))
    return stack, leaf, act, weights, residual


def test_down_combine_matches_oracle():
    print("moe_down_combine_mxfp4", flush=True)
    rng = np.random.default_rng(4)
    stack, leaf, act, weights, residual = _down(rng, 4)
    chosen = [6, 2, 0, 5]
    got = ops.moe_down_combine_mxfp4(to_device(act), leaf, _ids(chosen), f32_to_device(weights),
                                     to_device(residual))
    assert_bf16_close(bits_of(got), mxfp4.down_combine(act, stack, chosen, weights, residual),
                      min_exact=0.99)


def test_down_combine_gpt_oss_shape():
    print("moe_down_combine_mxfp4 gpt-oss-120b", flush=True)
    rng = np.random.default_rng(5)
    stack, leaf, act, weights, residual = _down(rng, 4, hidden=2880, inner=2880, experts=128)
    chosen = [17, 127, 64, 3]
    got = ops.moe_down_combine_mxfp4(to_device(act), leaf, _ids(chosen), f32_to_device(weights),
                                     to_device(residual))
    assert_bf16_close(bits_of(got), mxfp4.down_combine(act, stack, chosen, weights, residual),
                      min_exact=0.99)


@pytest.mark.parametrize("slots", [1, 16])
def test_down_combine_slots_no_bias_no_residual(slots):
    print(f"moe_down_combine_mxfp4 slots={slots}", flush=True)
    rng = np.random.default_rng(6 + slots)
    stack, leaf, act, weights, _ = _down(rng, slots, hidden=520, inner=3072, experts=20, bias=False)
    chosen = list(rng.integers(0, 20, size=slots))
    got = ops.moe_down_combine_mxfp4(to_device(act), leaf, _ids(chosen), f32_to_device(weights))
    assert_bf16_close(bits_of(got), mxfp4.down_combine(act, stack, chosen, weights, None), min_exact=0.99)


def test_down_combine_invalid_id_and_zero_weights():
    rng = np.random.default_rng(8)
    stack, leaf, act, weights, residual = _down(rng, 3)
    chosen = [2, -5, 7]
    got = ops.moe_down_combine_mxfp4(to_device(act), leaf, _ids(chosen), f32_to_device(weights),
                                     to_device(residual))
    assert_bf16_close(bits_of(got), mxfp4.down_combine(act, stack, chosen, weights, residual),
                      min_exact=0.99)
    zero = ops.moe_down_combine_mxfp4(to_device(act), leaf, _ids(chosen),
                                      f32_to_device(np.zeros(3, np.float32)), to_device(residual))
    assert np.array_equal(to_f32(bits_of(zero)), to_f32(residual))


def test_shape_checks_raise_before_launch():
    rng = np.random.default_rng(9)
    _, leaf = _leaf(rng, EXPERTS, 2 * INNER, HIDDEN)
    with pytest.raises(ValueError):
        ops.moe_gate_up_mxfp4(to_device(from_float(rng.standard_normal(HIDDEN + 32))), leaf, _ids([0]))
    _, dleaf = _leaf(rng, EXPERTS, HIDDEN, 4096)
    act = to_device(from_float(rng.standard_normal((2, 4096))))
    with pytest.raises(ValueError):                           # inner past the kernel's 3072
        ops.moe_down_combine_mxfp4(act, dleaf, _ids([0, 1]), f32_to_device(np.ones(2, np.float32)))

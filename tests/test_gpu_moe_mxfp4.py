"""HIP MXFP4 routed-expert kernels (csrc/moe_fp4.hip) against the oracle
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


@pytest.mark.parametrize("hidden", [32, 2048, 4096 + 32, 16384])
def test_gate_up_trip_counts(hidden):
    """One, two and more 64-chunk trips per lane (the runtime loop, odd trip counts)."""
    print(f"moe_gate_up_mxfp4 hidden={hidden}", flush=True)
    rng = np.random.default_rng(hidden)
    stack, leaf = _leaf(rng, 3, 2 * 96, hidden)
    x = from_float(rng.standard_normal(hidden))
    got = ops.moe_gate_up_mxfp4(to_device(x), leaf, _ids([2, 0]), limit=7.0)
    assert_bf16_close(bits_of(got), mxfp4.gate_up(x, stack, [2, 0], 7.0), min_exact=0.99)


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


@pytest.mark.parametrize("slots,hidden,inner", [(1, 520, 3072), (16, 522, 4096), (3, 64, 2048), (2, 7, 96)])
def test_down_combine_slots_no_bias_no_residual(slots, hidden, inner):
    """Row counts that leave the last workgroup short, one and two 64-chunk steps."""
    print(f"moe_down_combine_mxfp4 slots={slots} hidden={hidden} inner={inner}", flush=True)
    rng = np.random.default_rng(6 + slots)
    stack, leaf, act, weights, _ = _down(rng, slots, hidden=hidden, inner=inner, experts=20, bias=False)
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
    _, dleaf = _leaf(rng, EXPERTS, HIDDEN, 4128)
    act = to_device(from_float(rng.standard_normal((2, 4128))))
    with pytest.raises(ValueError):                           # inner past the kernel's 4096
        ops.moe_down_combine_mxfp4(act, dleaf, _ids([0, 1]), f32_to_device(np.ones(2, np.float32)))


def _switch_leaf(leaf):
    from mlx_omnia_amd.kernels.leaf import QuantizedSwitchLinearLeaf

    return QuantizedSwitchLinearLeaf(leaf.weight, leaf.scales, None, 32, 4, mode="mxfp4")


def test_facades_resolve_to_the_mxfp4_bindings_and_agree_with_the_core_chain():
    from mlx_omnia_amd.kernels.down_combine import DefaultDownCombine, DownCombine, HipMxfp4DownCombine
    from mlx_omnia_amd.kernels.gate_up import DefaultGateUp, GateUp, HipMxfp4GateUp

    rng = np.random.default_rng(10)
    _, g = _leaf(rng, EXPERTS, 2 * INNER, HIDDEN)
    _, d = _leaf(rng, EXPERTS, HIDDEN, INNER)
    gleaf, dleaf = _switch_leaf(g), _switch_leaf(d)
    declared = dict(hidden=HIDDEN, inner=INNER, activation="swiglu_oai", limit=7.0, bias=g.bias)
    gate_up = GateUp(gleaf, **declared)
    down = DownCombine(dleaf, hidden=HIDDEN, inner=INNER, bias=d.bias)
    assert isinstance(gate_up.strategy, HipMxfp4GateUp)
    assert isinstance(down.strategy, HipMxfp4DownCombine)
    core_gate_up = GateUp(gleaf, reference=True, **declared)
    core_down = DownCombine(dleaf, hidden=HIDDEN, inner=INNER, bias=d.bias, reference=True)
    assert isinstance(core_gate_up.strategy, DefaultGateUp)
    assert isinstance(core_down.strategy, DefaultDownCombine)
    # What the kernels do not bake goes to the Core chain: no bias, no clamp, silu, the
    # blocked layout, a shared expert.
    for change in (dict(bias=None), dict(limit=None), dict(activation="silu"), dict(layout="blocked"),
                   dict(shared=lambda row: row)):
        assert isinstance(GateUp(gleaf, **dict(declared, **change)).strategy, DefaultGateUp), change
    assert isinstance(DownCombine(dleaf, hidden=HIDDEN, inner=INNER).strategy, DefaultDownCombine)

    x = from_float(2 * rng.standard_normal(HIDDEN))
    chosen = torch.tensor([2, 7, 0, 5], dtype=torch.int32, device="cuda")
    act = gate_up(to_device(x), chosen)
    assert torch.equal(act, ops.moe_gate_up_mxfp4(to_device(x), g, chosen, limit=7.0))
    # The Core chain rounds 1.702 g to bf16 before the sigmoid: the same function, looser.
    core_act = core_gate_up(to_device(x), chosen)
    np.testing.assert_allclose(act.float().cpu().numpy(), core_act.float().cpu().numpy(), rtol=0.06, atol=0.02)
    weights = torch.tensor([0.4, 0.3, 0.2, 0.1], dtype=torch.float32, device="cuda")
    residual = to_device(from_float(rng.standard_normal(HIDDEN)))
    got = down(act, chosen, weights, residual)
    assert torch.equal(got, ops.moe_down_combine_mxfp4(act, d, chosen, weights, residual))
    core = core_down(act, chosen, weights.to(torch.bfloat16), residual).float().cpu().numpy()
    # The Core chain rounds each row before the bias add and each weighted row to bf16: a
    # few ulps of the largest term, so the bound is relative to the output's scale.
    assert np.abs(got.float().cpu().numpy() - core).max() <= 4 * 2.0 ** -8 * np.abs(core).max()


def test_down_facade_hands_more_than_16_slots_to_the_core_chain():
    from mlx_omnia_amd.kernels.down_combine import DownCombine, HipMxfp4DownCombine

    rng = np.random.default_rng(11)
    stack, d = _leaf(rng, EXPERTS, HIDDEN, INNER)
    down = DownCombine(_switch_leaf(d), hidden=HIDDEN, inner=INNER, bias=d.bias)
    assert isinstance(down.strategy, HipMxfp4DownCombine)
    ids = list(rng.integers(0, EXPERTS, size=20))
    act = from_float(rng.standard_normal((20, INNER)))
    weights = np.full(20, 0.05, dtype=np.float32)
    got = down(to_device(act), _ids(ids), f32_to_device(weights), None).to(torch.bfloat16)
    # The Core chain rounds each row before the bias add and sums in torch's order: within
    # the bf16 bar (2 ulps of the output's scale), about 40% bit-identical at this shape.
    assert_bf16_close(bits_of(got), mxfp4.down_combine(act, stack, ids, weights, None), min_exact=0.3)


def test_golden_fixture():
    golden = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "moe_mxfp4.npz")

    def leaf(name):
        return ops.Mxfp4Leaf(torch.from_numpy(golden[f"{name}_weight"].view(np.int32)).cuda(),
                             torch.from_numpy(golden[f"{name}_scales"]).cuda(), to_device(golden[f"{name}_bias"]))

    chosen = torch.from_numpy(golden["chosen"]).cuda()
    act = ops.moe_gate_up_mxfp4(to_device(golden["x"]), leaf("gate_up"), chosen, limit=float(golden["limit"]))
    assert_bf16_close(bits_of(act), golden["act"], min_exact=0.99)
    out = ops.moe_down_combine_mxfp4(to_device(golden["act"]), leaf("down"), chosen,
                                     f32_to_device(golden["weights"]), to_device(golden["residual"]))
    assert_bf16_close(bits_of(out), golden["out"], min_exact=0.99)

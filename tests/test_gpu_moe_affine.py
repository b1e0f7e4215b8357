"""HIP affine-quantized routed-expert kernels (csrc/moe_affine.hip) against the oracle
(oracle/affine.py).

Mirrors the reference's tests of the affine gate-up and down-combine kernels
(tests/test_kernel_moe_gemv.py): every bit width the decoder switches on (2, 3, 4, 5, 6,
8) and every group size, the clamp, the shared expert decoded on its own width and group
in the last slot, and the same smallest-twice-over shapes (hidden 1024, inner 512). Beyond
those: Qwen3-30B-A3B's routed MLP at 4 bits (hidden 2048, inner 768, 128 experts, top-8),
invalid expert ids, no residual, 1 and 16 slots.

The kernels sum in fp32 in their own order (and, below 8 bits, through bf16 128 + q pairs
whose offset comes back out through the bias term); the oracle rounds the exact dot
product once. Bar: the north-star bf16 bar (assert_bf16_close) with at least 99% of the
outputs bit-identical.

Stacks are random words (every bit pattern is a valid value) with scales of the size a
quantized checkpoint has (a row's dot product of order one) and biases centring them.
"""

import numpy as np
import pytest
import torch

from mlx_omnia_amd.runtime import ops
from oracle import affine
from oracle.bf16 import from_float, to_f32
from util import assert_bf16_close, bits_of, f32_to_device, to_device

pytestmark = pytest.mark.gpu

HIDDEN, INNER, EXPERTS = 1024, 512, 8


def _leaf(rng, lead, rows, features, bits, group):
    """(oracle Stack, device AffineLeaf) of random words, scales and centring biases."""
    words = rng.integers(0, 1 << 32, size=lead + (rows, features * bits // 32), dtype=np.uint64)
    words = words.astype(np.uint32)
    scale = 4.0 / ((1 << bits) * np.sqrt(features))
    shape = lead + (rows, features // group)
    s = from_float(scale * (0.5 + rng.random(shape)))
    b = from_float(-to_f32(s) * ((1 << bits) - 1) / 2 * (0.8 + 0.4 * rng.random(shape)))
    stack = affine.Stack(words, s, b, group, bits)
    leaf = ops.AffineLeaf(torch.from_numpy(words.view(np.int32)).cuda(), to_device(s), to_device(b),
                          bits, group)
    return stack, leaf


def _ids(values):
    return torch.tensor(values, dtype=torch.int32, device="cuda")


@pytest.mark.parametrize("group", affine.GROUPS)
@pytest.mark.parametrize("bits", affine.WIDTHS)
def test_gate_up_matches_oracle(bits, group):
    print(f"moe_gate_up_affine bits={bits} group={group}", flush=True)
    rng = np.random.default_rng(bits * 1000 + group)
    stack, leaf = _leaf(rng, (EXPERTS,), 2 * INNER, HIDDEN, bits, group)
    x = from_float(rng.standard_normal(HIDDEN))
    chosen = [5, 0, 7, 2]
    got = ops.moe_gate_up_affine(to_device(x), leaf, _ids(chosen))
    want = affine.gate_up(x, stack, chosen)
    assert_bf16_close(bits_of(got), want, min_exact=0.99)


def test_gate_up_qwen3_30b_shape():
    print("moe_gate_up_affine Qwen3-30B-A3B 4-bit g64", flush=True)
    rng = np.random.default_rng(30)
    stack, leaf = _leaf(rng, (128,), 2 * 768, 2048, 4, 64)
    x = from_float(rng.standard_normal(2048))
    chosen = [17, 3, 127, 64, 0, 99, 41, 8]
    got = ops.moe_gate_up_affine(to_device(x), leaf, _ids(chosen))
    assert_bf16_close(bits_of(got), affine.gate_up(x, stack, chosen), min_exact=0.99)


@pytest.mark.parametrize("bits", [2, 4, 6, 8])
def test_gate_up_clamp(bits):
    print(f"moe_gate_up_affine clamp bits={bits}", flush=True)
    rng = np.random.default_rng(40 + bits)
    stack, leaf = _leaf(rng, (EXPERTS,), 2 * INNER, HIDDEN, bits, 64)
    x = from_float(3 * rng.standard_normal(HIDDEN))
    limit = 0.5
    got = bits_of(ops.moe_gate_up_affine(to_device(x), leaf, _ids([1, 6]), limit=limit))
    want = affine.gate_up(x, stack, [1, 6], limit=limit)
    assert_bf16_close(got, want, min_exact=0.99)
    assert not np.array_equal(want, affine.gate_up(x, stack, [1, 6]))  # the limit bites


@pytest.mark.parametrize("widths", [(3, 8), (8, 3), (4, 2), (2, 5)])
def test_shared_slot_decodes_on_its_own_width(widths):
    bits, shared_bits = widths
    print(f"moe affine shared slot bits={bits} shared_bits={shared_bits}", flush=True)
    rng = np.random.default_rng(50 + bits * 10 + shared_bits)
    stack, leaf = _leaf(rng, (EXPERTS,), 2 * INNER, HIDDEN, bits, 64)
    sstack, sleaf = _leaf(rng, (), 2 * INNER, HIDDEN, shared_bits, 128)
    x = from_float(rng.standard_normal(HIDDEN))
    chosen = [4, 1, 2, 1000]      # the shared slot's index is never read
    act = ops.moe_gate_up_affine(to_device(x), leaf, _ids(chosen), shared=sleaf)
    want_act = affine.gate_up(x, stack, chosen, shared=sstack)
    assert_bf16_close(bits_of(act), want_act, min_exact=0.99)

    dstack, dleaf = _leaf(rng, (EXPERTS,), HIDDEN, INNER, bits, 64)
    sdstack, sdleaf = _leaf(rng, (), HIDDEN, INNER, shared_bits, 128)
    weights = np.array([0.4, 0.3, 0.2, 0.1], dtype=np.float32)
    residual = from_float(rng.standard_normal(HIDDEN))
    got = ops.moe_down_combine_affine(to_device(want_act), dleaf, _ids(chosen), f32_to_device(weights),
                                      to_device(residual), shared=sdleaf)
    want = affine.down_combine(want_act, dstack, chosen, weights, residual, shared=sdstack)
    assert_bf16_close(bits_of(got), want, min_exact=0.99)


def test_gate_up_invalid_ids_give_zeros():
    rng = np.random.default_rng(60)
    stack, leaf = _leaf(rng, (EXPERTS,), 2 * INNER, HIDDEN, 4, 32)
    x = from_float(rng.standard_normal(HIDDEN))
    got = bits_of(ops.moe_gate_up_affine(to_device(x), leaf, _ids([-1, 3, EXPERTS])))
    assert np.all(got[0] == 0) and np.all(got[2] == 0)
    assert_bf16_close(got[1:2], affine.gate_up(x, stack, [3]), min_exact=0.99)


def _down_case(rng, bits, group, slots, hidden=HIDDEN, inner=INNER, experts=EXPERTS):
    stack, leaf = _leaf(rng, (experts,), hidden, inner, bits, group)
    act = from_float(rng.standard_normal((slots, inner)))
    weights = rng.dirichlet(np.ones(slots)).astype(np.float32)
    residual = from_float(rng.standard_normal(hidden))
    return stack, leaf, act, weights, residual


@pytest.mark.parametrize("group", affine.GROUPS)
@pytest.mark.parametrize("bits", affine.WIDTHS)
def test_down_combine_matches_oracle(bits, group):
    print(f"moe_down_combine_affine bits={bits} group={group}", flush=True)
    rng = np.random.default_rng(70 + bits * 1000 + group)
    stack, leaf, act, weights, residual = _down_case(rng, bits, group, 4)
    chosen = [6, 2, 0, 5]
    got = ops.moe_down_combine_affine(to_device(act), leaf, _ids(chosen), f32_to_device(weights),
                                      to_device(residual))
    want = affine.down_combine(act, stack, chosen, weights, residual)
    assert_bf16_close(bits_of(got), want, min_exact=0.99)


def test_down_combine_qwen3_30b_shape():
    print("moe_down_combine_affine Qwen3-30B-A3B 4-bit g64", flush=True)
    rng = np.random.default_rng(80)
    stack, leaf, act, weights, residual = _down_case(rng, 4, 64, 8, hidden=2048, inner=768, experts=128)
    chosen = [17, 3, 127, 64, 0, 99, 41, 8]
    got = ops.moe_down_combine_affine(to_device(act), leaf, _ids(chosen), f32_to_device(weights),
                                      to_device(residual))
    assert_bf16_close(bits_of(got), affine.down_combine(act, stack, chosen, weights, residual),
                      min_exact=0.99)


@pytest.mark.parametrize("slots", [1, 16])
def test_down_combine_slot_counts_and_no_residual(slots):
    print(f"moe_down_combine_affine slots={slots}", flush=True)
    rng = np.random.default_rng(90 + slots)
    stack, leaf, act, weights, _ = _down_case(rng, 4, 32, slots, hidden=520, inner=1536, experts=20)
    chosen = list(rng.integers(0, 20, size=slots))
    got = ops.moe_down_combine_affine(to_device(act), leaf, _ids(chosen), f32_to_device(weights))
    assert_bf16_close(bits_of(got), affine.down_combine(act, stack, chosen, weights, None),
                      min_exact=0.99)


def test_down_combine_invalid_id_and_zero_weights():
    rng = np.random.default_rng(100)
    stack, leaf, act, weights, residual = _down_case(rng, 8, 128, 3)
    chosen = [2, -5, 7]
    got = ops.moe_down_combine_affine(to_device(act), leaf, _ids(chosen), f32_to_device(weights),
                                      to_device(residual))
    assert_bf16_close(bits_of(got), affine.down_combine(act, stack, chosen, weights, residual),
                      min_exact=0.99)
    zero = ops.moe_down_combine_affine(to_device(act), leaf, _ids(chosen),
                                       f32_to_device(np.zeros(3, np.float32)), to_device(residual))
    assert np.array_equal(to_f32(bits_of(zero)), to_f32(residual))


def test_shape_checks_raise_before_launch():
    rng = np.random.default_rng(110)
    _, leaf = _leaf(rng, (EXPERTS,), 2 * INNER, HIDDEN, 4, 64)
    x = to_device(from_float(rng.standard_normal(HIDDEN + 32)))
    with pytest.raises(ValueError):
        ops.moe_gate_up_affine(x, leaf, _ids([0]))          # hidden mismatch
    bad = ops.AffineLeaf(leaf.weight, leaf.scales, leaf.biases, 4, 16)
    with pytest.raises(ValueError):
        ops.moe_gate_up_affine(to_device(from_float(rng.standard_normal(HIDDEN))), bad, _ids([0]))
    _, dleaf = _leaf(rng, (EXPERTS,), HIDDEN, 2048, 4, 64)
    act = to_device(from_float(rng.standard_normal((2, 2048))))
    with pytest.raises(ValueError):                           # inner past the kernel's 1536
        ops.moe_down_combine_affine(act, dleaf, _ids([0, 1]), f32_to_device(np.ones(2, np.float32)))


def test_facades_resolve_to_the_affine_bindings_and_agree_with_the_core_chain():
    from mlx_omnia_amd.kernels.down_combine import (DefaultDownCombine, DownCombine,
                                                    HipAffineDownCombine)
    from mlx_omnia_amd.kernels.gate_up import DefaultGateUp, GateUp, HipAffineGateUp
    from mlx_omnia_amd.kernels.leaf import QuantizedLinearLeaf, QuantizedSwitchLinearLeaf

    print("moe affine facades", flush=True)
    rng = np.random.default_rng(120)
    gstack, g = _leaf(rng, (EXPERTS,), 2 * INNER, HIDDEN, 4, 64)
    dstack, d = _leaf(rng, (EXPERTS,), HIDDEN, INNER, 4, 64)
    sstack, s = _leaf(rng, (), 2 * INNER, HIDDEN, 8, 128)
    sdstack, sd = _leaf(rng, (), HIDDEN, INNER, 8, 128)
    gleaf = QuantizedSwitchLinearLeaf(g.weight, g.scales, g.biases, 64, 4)
    dleaf = QuantizedSwitchLinearLeaf(d.weight, d.scales, d.biases, 64, 4)
    shared_gate = QuantizedLinearLeaf(s.weight, s.scales, s.biases, 128, 8)
    shared_down = QuantizedLinearLeaf(sd.weight, sd.scales, sd.biases, 128, 8)
    gate_up = GateUp(gleaf, hidden=HIDDEN, inner=INNER, shared=shared_gate)
    down = DownCombine(dleaf, hidden=HIDDEN, inner=INNER, shared=shared_down)
    assert isinstance(gate_up.strategy, HipAffineGateUp)
    assert isinstance(down.strategy, HipAffineDownCombine)
    core_gate_up = GateUp(gleaf, hidden=HIDDEN, inner=INNER, shared=shared_gate, reference=True)
    core_down = DownCombine(dleaf, hidden=HIDDEN, inner=INNER, shared=shared_down, reference=True)
    assert isinstance(core_gate_up.strategy, DefaultGateUp)
    assert isinstance(core_down.strategy, DefaultDownCombine)
    # A layout or a mode the kernels do not decode goes to the Core chain.
    assert isinstance(GateUp(gleaf, hidden=HIDDEN, inner=INNER, layout="blocked").strategy, DefaultGateUp)
    mx = QuantizedSwitchLinearLeaf(g.weight, g.scales, None, 64, 4, mode="mxfp4")
    assert isinstance(GateUp(mx, hidden=HIDDEN, inner=INNER).strategy, DefaultGateUp)

    x = from_float(rng.standard_normal(HIDDEN))
    chosen = torch.tensor([2, 7, 0, 0], dtype=torch.int32, device="cuda")
    act = gate_up(to_device(x), chosen)
    want_act = affine.gate_up(x, gstack, [2, 7, 0, 0], shared=sstack)
    assert_bf16_close(bits_of(act), want_act, min_exact=0.99)
    assert_bf16_close(bits_of(core_gate_up(to_device(x), chosen)), want_act, min_exact=0.97)

    weights = torch.tensor([0.4, 0.3, 0.2, 0.1], dtype=torch.bfloat16, device="cuda")
    residual = from_float(rng.standard_normal(HIDDEN))
    out = down(act, chosen, weights, to_device(residual))
    want = affine.down_combine(bits_of(act), dstack, [2, 7, 0, 0], weights.float().cpu().numpy(),
                               residual, shared=sdstack)
    assert_bf16_close(bits_of(out), want, min_exact=0.99)
    core = core_down(act, chosen, weights, to_device(residual))
    assert_bf16_close(bits_of(core), want, min_exact=0.8)


def test_down_facade_hands_more_than_16_slots_to_the_core_chain():
    from mlx_omnia_amd.kernels.down_combine import DownCombine, HipAffineDownCombine
    from mlx_omnia_amd.kernels.leaf import QuantizedSwitchLinearLeaf

    rng = np.random.default_rng(130)
    dstack, d = _leaf(rng, (EXPERTS,), HIDDEN, INNER, 4, 32)
    down = DownCombine(QuantizedSwitchLinearLeaf(d.weight, d.scales, d.biases, 32, 4), hidden=HIDDEN,
                       inner=INNER)
    assert isinstance(down.strategy, HipAffineDownCombine)
    chosen = list(rng.integers(0, EXPERTS, size=20))
    act = from_float(rng.standard_normal((20, INNER)))
    weights = np.full(20, 0.05, dtype=np.float32)
    out = down(to_device(act), torch.tensor(chosen, dtype=torch.int32, device="cuda"),
               f32_to_device(weights), None)
    want = affine.down_combine(act, dstack, chosen, weights, None)
    assert_bf16_close(bits_of(out.to(torch.bfloat16)), want, min_exact=0.5)


def test_golden_fixture():
    golden = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "moe_affine.npz")

    def leaf(name):
        bits, group = (int(v) for v in golden[f"{name}_format"])
        return ops.AffineLeaf(torch.from_numpy(golden[f"{name}_weight"].view(np.int32)).cuda(),
                              to_device(golden[f"{name}_scales"]), to_device(golden[f"{name}_biases"]),
                              bits, group)

    chosen = torch.from_numpy(golden["chosen"]).cuda()
    act = ops.moe_gate_up_affine(to_device(golden["x"]), leaf("gate_up"), chosen, shared=leaf("shared_gate_up"))
    assert_bf16_close(bits_of(act), golden["act"], min_exact=0.99)
    out = ops.moe_down_combine_affine(to_device(golden["act"]), leaf("down"), chosen,
                                      f32_to_device(golden["weights"]), to_device(golden["residual"]),
                                      shared=leaf("shared_down"))
    assert_bf16_close(bits_of(out), golden["out"], min_exact=0.99)

"""HIP NVFP4 routed-expert kernels (csrc/moe_fp4.hip) against the oracle (oracle/nvfp4.py).

Mirrors the reference's nvfp4 strategies (core/kernels/gate_up/nvfp4.py,
core/kernels/down_combine/nvfp4.py): the interleaved layout, e4m3 scales per 16 values,
the plain SwiGLU chain, no bias. Shapes: Qwen3-30B-A3B's routed MLP (hidden 2048, inner
768, 128 experts, top-8) and small ones; negative and all-ones scale codes; invalid
expert ids; no residual; 1 and 16 slots; one, two and more 64-chunk trips.

Bar: the north-star bf16 bar (assert_bf16_close) with at least 99% of the outputs
bit-identical.
"""

import numpy as np
import pytest
import torch

from mlx_omnia_amd.runtime import ops
from oracle import nvfp4
from oracle.bf16 import from_float, to_f32
from util import assert_bf16_close, bits_of, f32_to_device, to_device

pytestmark = pytest.mark.gpu


def _leaf(rng, experts, rows, features, special=False):
    words = rng.integers(0, 1 << 32, size=(experts, rows, features // 8), dtype=np.uint64).astype(np.uint32)
    scales = rng.integers(0x18, 0x28, size=(experts, rows, features // 16)).astype(np.uint8)
    if special:   # negative scales, the subnormals and mlx's +-480 codes
        scales[..., 0] = 0x7F
        scales[..., 1] = 0xB0
        scales[..., 2] = 0x05
        scales[..., 3] = 0xFF
    stack = nvfp4.Stack(words, scales)
    leaf = ops.Nvfp4Leaf(torch.from_numpy(words.view(np.int32)).cuda(), torch.from_numpy(scales).cuda(), None)
    return stack, leaf


def _ids(values):
    return torch.tensor(values, dtype=torch.int32, device="cuda")


@pytest.mark.parametrize("hidden,inner,special", [(2048, 768, False), (512, 96, True), (32, 64, False),
                                                   (4096 + 32, 64, False), (16384, 32, False)])
def test_gate_up_matches_oracle(hidden, inner, special):
    print(f"moe_gate_up_nvfp4 hidden={hidden} inner={inner}", flush=True)
    rng = np.random.default_rng(hidden + inner)
    experts = 128 if hidden == 2048 else 4
    stack, leaf = _leaf(rng, experts, 2 * inner, hidden, special)
    x = from_float(rng.standard_normal(hidden) / (8 if special else 1))
    chosen = list(rng.choice(experts, size=min(8, experts), replace=False))
    got = ops.moe_gate_up_nvfp4(to_device(x), leaf, _ids(chosen))
    assert_bf16_close(bits_of(got), nvfp4.gate_up(x, stack, chosen), min_exact=0.99)


def test_gate_up_invalid_ids_give_zeros():
    rng = np.random.default_rng(3)
    stack, leaf = _leaf(rng, 4, 128, 256)
    x = from_float(rng.standard_normal(256))
    got = bits_of(ops.moe_gate_up_nvfp4(to_device(x), leaf, _ids([-1, 3, 4])))
    assert np.all(got[0] == 0) and np.all(got[2] == 0)
    assert_bf16_close(got[1:2], nvfp4.gate_up(x, stack, [3]), min_exact=0.99)


@pytest.mark.parametrize("slots,hidden,inner,experts", [(8, 2048, 768, 128), (1, 520, 4096, 6), (16, 66, 2048, 20),
                                                         (3, 7, 96, 4)])
def test_down_combine_matches_oracle(slots, hidden, inner, experts):
    print(f"moe_down_combine_nvfp4 slots={slots} hidden={hidden} inner={inner}", flush=True)
    rng = np.random.default_rng(slots + hidden)
    stack, leaf = _leaf(rng, experts, hidden, inner, special=slots == 3)
    act = from_float(rng.standard_normal((slots, inner)))
    weights = rng.dirichlet(np.ones(slots)).astype(np.float32)
    residual = from_float(rng.standard_normal(hidden)) if slots != 1 else None
    chosen = list(rng.integers(0, experts, size=slots))
    if slots == 3:
        chosen[1] = -2   # an invalid id contributes nothing
    got = ops.moe_down_combine_nvfp4(to_device(act), leaf, _ids(chosen), f32_to_device(weights),
                                     None if residual is None else to_device(residual))
    assert_bf16_close(bits_of(got), nvfp4.down_combine(act, stack, chosen, weights, residual), min_exact=0.99)


def test_facades_resolve_to_the_nvfp4_bindings():
    from mlx_omnia_amd.kernels.down_combine import DefaultDownCombine, DownCombine, HipNvfp4DownCombine
    from mlx_omnia_amd.kernels.gate_up import DefaultGateUp, GateUp, HipNvfp4GateUp
    from mlx_omnia_amd.kernels.leaf import QuantizedSwitchLinearLeaf

    rng = np.random.default_rng(10)
    gstack, g = _leaf(rng, 6, 2 * 128, 512)
    dstack, d = _leaf(rng, 6, 512, 128)
    gleaf = QuantizedSwitchLinearLeaf(g.weight, g.scales, None, 16, 4, mode="nvfp4")
    dleaf = QuantizedSwitchLinearLeaf(d.weight, d.scales, None, 16, 4, mode="nvfp4")
    gate_up = GateUp(gleaf, hidden=512, inner=128)
    down = DownCombine(dleaf, hidden=512, inner=128)
    assert isinstance(gate_up.strategy, HipNvfp4GateUp)
    assert isinstance(down.strategy, HipNvfp4DownCombine)
    for change in (dict(limit=7.0), dict(activation="swiglu_oai", limit=7.0), dict(layout="blocked"),
                   dict(bias=torch.zeros(6, 256, dtype=torch.bfloat16, device="cuda"))):
        assert isinstance(GateUp(gleaf, hidden=512, inner=128, **change).strategy, DefaultGateUp), change
    assert isinstance(DownCombine(dleaf, hidden=512, inner=128, layout="blocked").strategy, DefaultDownCombine)
    x = from_float(rng.standard_normal(512))
    chosen = _ids([5, 0, 3])
    act = gate_up(to_device(x), chosen)
    assert torch.equal(act, ops.moe_gate_up_nvfp4(to_device(x), g, chosen))
    core = GateUp(gleaf, hidden=512, inner=128, reference=True)(to_device(x), chosen)
    assert_bf16_close(bits_of(act), bits_of(core), min_exact=0.95)
    weights = torch.tensor([0.5, 0.3, 0.2], dtype=torch.float32, device="cuda")
    residual = to_device(from_float(rng.standard_normal(512)))
    out = down(act, chosen, weights, residual)
    assert torch.equal(out, ops.moe_down_combine_nvfp4(act, d, chosen, weights, residual))
    want = nvfp4.down_combine(bits_of(act), dstack, [5, 0, 3], weights.cpu().numpy(), bits_of(residual))
    assert_bf16_close(bits_of(out), want, min_exact=0.99)


def test_golden_fixture():
    golden = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "moe_nvfp4.npz")

    def leaf(name):
        return ops.Nvfp4Leaf(torch.from_numpy(golden[f"{name}_weight"].view(np.int32)).cuda(),
                             torch.from_numpy(golden[f"{name}_scales"]).cuda(), None)

    chosen = torch.from_numpy(golden["chosen"]).cuda()
    act = ops.moe_gate_up_nvfp4(to_device(golden["x"]), leaf("gate_up"), chosen)
    assert_bf16_close(bits_of(act), golden["act"], min_exact=0.99)
    out = ops.moe_down_combine_nvfp4(to_device(golden["act"]), leaf("down"), chosen,
                                     f32_to_device(golden["weights"]), to_device(golden["residual"]))
    assert_bf16_close(bits_of(out), golden["out"], min_exact=0.99)


def test_shape_checks_raise_before_launch():
    rng = np.random.default_rng(9)
    _, leaf = _leaf(rng, 4, 128, 256)
    with pytest.raises(ValueError):
        ops.moe_gate_up_nvfp4(to_device(from_float(rng.standard_normal(288))), leaf, _ids([0]))
    with pytest.raises(ValueError):   # NVFP4 stacks carry no bias
        ops.moe_gate_up_nvfp4(to_device(from_float(rng.standard_normal(256))),
                              ops.Nvfp4Leaf(leaf.weight, leaf.scales, torch.zeros(4, 128, dtype=torch.bfloat16,
                                                                                   device="cuda")), _ids([0]))


def _ranked(keys, top_k):
    """Ascending ordinal keys, equal keys to the lower index (a stable sort)."""
    return list(np.argsort(keys.astype(np.uint64), kind="stable")[:top_k])


@pytest.mark.parametrize("experts,top_k,hidden", [(128, 8, 2048), (200, 8, 256), (1024, 4, 512), (64, 64, 96), (32, 1, 32)])
def test_ordinal_routing_in_the_kernel(experts, top_k, hidden):
    print(f"moe_gate_up_nvfp4_ordinal experts={experts} top_k={top_k}", flush=True)
    rng = np.random.default_rng(experts + top_k)
    stack, leaf = _leaf(rng, experts, 2 * 64, hidden)
    keys = rng.integers(0, 1 << 32, size=experts, dtype=np.uint64).astype(np.uint32)
    keys[5::7] = keys[3]                                  # ties, resolved to the lower index
    keys[1] = np.uint32(0xFFFFFFF0)                       # above 2^31: compared unsigned
    x = from_float(rng.standard_normal(hidden))
    got = ops.moe_gate_up_nvfp4_ordinal(to_device(x), leaf, torch.from_numpy(keys).cuda(), top_k)
    chosen = _ranked(keys, top_k)
    assert_bf16_close(bits_of(got), nvfp4.gate_up(x, stack, chosen), min_exact=0.99)
    by_index = ops.moe_gate_up_nvfp4(to_device(x), leaf, _ids(chosen))
    assert torch.equal(got, by_index)


def test_ordinal_keys_must_be_unsigned():
    """The op takes uint32 keys only; through the facade, int32 keys go to the Core chain,
    which sorts them as signed (as mx.argsort would), a negative key ranking first."""
    rng = np.random.default_rng(3)
    experts, hidden = 32, 64
    stack, leaf = _leaf(rng, experts, 2 * 64, hidden)
    keys = rng.integers(0, 1 << 20, size=experts).astype(np.int32)
    keys[9] = -5
    x = from_float(rng.standard_normal(hidden))
    with pytest.raises(ValueError, match="uint32"):
        ops.moe_gate_up_nvfp4_ordinal(to_device(x), leaf, torch.from_numpy(keys).cuda(), 4)
    signed = list(np.argsort(keys.astype(np.int64), kind="stable")[:4])
    assert signed[0] == 9


def test_ordinal_facade():
    from mlx_omnia_amd.kernels.gate_up import GateUp, HipNvfp4GateUp, OrdinalRouting
    from mlx_omnia_amd.kernels.leaf import QuantizedSwitchLinearLeaf

    rng = np.random.default_rng(12)
    _, g = _leaf(rng, 64, 2 * 128, 256)
    gleaf = QuantizedSwitchLinearLeaf(g.weight, g.scales, None, 16, 4, mode="nvfp4")
    gate_up = GateUp(gleaf, hidden=256, inner=128, routing=OrdinalRouting(top_k=6))
    assert isinstance(gate_up.strategy, HipNvfp4GateUp)
    keys = rng.permutation(64).astype(np.uint32)
    x = to_device(from_float(rng.standard_normal(256)))
    got = gate_up(x, torch.from_numpy(keys).cuda())
    core = GateUp(gleaf, hidden=256, inner=128, routing=OrdinalRouting(top_k=6), reference=True)(
        x, torch.from_numpy(keys.astype(np.int64)).cuda())
    assert_bf16_close(bits_of(got), bits_of(core), min_exact=0.95)
    # int32 keys take the Core chain, which sorts them as signed integers.
    signed = gate_up(x, torch.from_numpy(keys.astype(np.int32)).cuda())
    assert torch.equal(signed, core)

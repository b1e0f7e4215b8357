"""The packed NVFP4 down/combine (`omnia_moe_down_combine_nvfp4_shared`, csrc/moe_fp4.hip)
against the oracle (oracle/nvfp4.py `down_combine_shared`).

Mirrors the reference's `Nvfp4PackedDownCombine` (core/kernels/down_combine/
nvfp4_packed.py): the routed slots and the shared stack on the last slot (unweighted),
several tokens per dispatch, the bf16 epilogue. Shapes: Qwen3-Next-80B-A3B's sparse
block (hidden 2048, inner 512, 512 experts, top-10 plus the shared expert), the
reference test's (hidden 64, inner 512, 8 experts, top-4, one and two tokens), and small
ones reaching every lane count (16, 32, 64 lanes across a row), more slots than waves
(21), a short last row tile, invalid ids, signed and all-ones scale codes, and no routed
slot at all.

Bar: the north-star bf16 bar (assert_bf16_close) with at least 99% of the outputs
bit-identical.
"""

import numpy as np
import pytest
import torch

from mlx_omnia_amd.runtime import ops
from oracle import nvfp4
from oracle.bf16 import from_float
from util import assert_bf16_close, bits_of, to_device

pytestmark = pytest.mark.gpu


def _stack(rng, experts, rows, features, *, paired=True, special=False):
    words = rng.integers(0, 1 << 32, size=(experts, rows, features // 8), dtype=np.uint64).astype(np.uint32)
    scales = rng.integers(0x18, 0x28, size=(experts, rows, features // 16)).astype(np.uint8)
    if paired:
        scales[..., 1::2] = scales[..., 0::2]
    if special:   # signed, subnormal and mlx's +-480 codes (the kernel reads any plane)
        scales[..., 0] = 0x7F
        scales[..., 1] = 0xB0
        scales[..., 2] = 0x05
        scales[..., -1] = 0xFF
    return nvfp4.Stack(words, scales)


def _leaf(stack):
    return ops.Nvfp4Leaf(torch.from_numpy(stack.weight.view(np.int32)).cuda(),
                         torch.from_numpy(stack.scales).cuda(), None)


def _run(seed, tokens, top_k, hidden, inner, experts, *, special=False, invalid=False):
    rng = np.random.default_rng(seed)
    routed = _stack(rng, experts, hidden, inner, special=special)
    shared = _stack(rng, 1, hidden, inner, special=special)
    act = from_float(rng.standard_normal((tokens, top_k + 1, inner)))
    chosen = rng.integers(0, experts, size=(tokens, top_k)).astype(np.int32)
    if invalid and top_k:
        chosen[0, 0] = -3
        chosen[-1, -1] = experts
    weights = rng.dirichlet(np.ones(max(top_k, 1)), size=tokens)[:, :top_k].astype(np.float32)
    residual = from_float(rng.standard_normal((tokens, hidden)))
    got = ops.moe_down_combine_nvfp4_shared(
        to_device(act), _leaf(routed), _leaf(nvfp4.Stack(shared.weight[0], shared.scales[0])),
        torch.from_numpy(chosen).cuda(), torch.from_numpy(weights).cuda(), to_device(residual))
    want = nvfp4.down_combine_shared(act, routed, nvfp4.Stack(shared.weight[0], shared.scales[0]),
                                     chosen, weights, residual)
    return bits_of(got), want


@pytest.mark.parametrize("tokens,top_k,hidden,inner,experts", [
    (1, 10, 2048, 512, 512),    # Qwen3-Next-80B-A3B
    (1, 4, 64, 512, 8),         # the reference test's shape
    (2, 4, 64, 512, 8),
    (5, 20, 100, 96, 6),        # 16 lanes, 21 slots on 16 waves, a short last tile
    (3, 3, 40, 1024, 5),        # 32 lanes
    (2, 1, 24, 2048, 3),        # 64 lanes
    (2, 0, 16, 512, 1),         # the shared slot alone
])
def test_matches_oracle(tokens, top_k, hidden, inner, experts):
    print(f"moe_down_combine_nvfp4_shared tokens={tokens} top_k={top_k} hidden={hidden} inner={inner}",
          flush=True)
    got, want = _run(tokens * 100 + top_k, tokens, top_k, hidden, inner, experts)
    assert got.shape == (tokens, hidden)
    assert_bf16_close(got, want, min_exact=0.99)


def test_invalid_ids_and_special_scales():
    got, want = _run(7, 3, 6, 72, 512, 9, special=True, invalid=True)
    assert_bf16_close(got, want, min_exact=0.99)


def _facade_case(seed, tokens, top_k, *, paired=True, with_shared=True):
    from mlx_omnia_amd.kernels.leaf import QuantizedLinearLeaf, QuantizedSwitchLinearLeaf

    rng = np.random.default_rng(seed)
    hidden, inner, experts = 256, 512, 16
    routed = _stack(rng, experts, hidden, inner, paired=paired)
    routed.scales[0, 0, 1] = 0x21   # the quantizer's first span, which the certificate allows
    shared = _stack(rng, 1, hidden, inner)
    leaf = QuantizedSwitchLinearLeaf(torch.from_numpy(routed.weight.view(np.int32)).cuda(),
                                     torch.from_numpy(routed.scales).cuda(), None, 16, 4, mode="nvfp4")
    shared_leaf = QuantizedLinearLeaf(torch.from_numpy(shared.weight[0].view(np.int32)).cuda(),
                                      torch.from_numpy(shared.scales[0]).cuda(), None, 16, 4, mode="nvfp4")
    act = from_float(rng.standard_normal((tokens, top_k + 1, inner)))
    chosen = np.concatenate([rng.integers(0, experts, size=(tokens, top_k)), np.zeros((tokens, 1))], axis=1)
    weights = np.concatenate([rng.dirichlet(np.ones(top_k), size=tokens), np.full((tokens, 1), 3.0)], axis=1)
    residual = from_float(rng.standard_normal((tokens, hidden)))
    return (routed, shared, leaf, shared_leaf if with_shared else None, act, chosen.astype(np.uint32),
            weights.astype(np.float32), residual)


def test_facade_binds_the_packed_strategy_for_a_certified_pair():
    from mlx_omnia_amd.kernels.down_combine import DownCombine, HipNvfp4PackedDownCombine

    routed, shared, leaf, shared_leaf, act, chosen, weights, residual = _facade_case(11, 3, 8)
    facade = DownCombine(leaf, hidden=256, inner=512, shared=shared_leaf)
    assert isinstance(facade.strategy, HipNvfp4PackedDownCombine)
    got = facade(to_device(act), torch.from_numpy(chosen.astype(np.int64)).cuda(),
                 torch.from_numpy(weights).cuda(), to_device(residual))
    want = nvfp4.down_combine_shared(act, routed, nvfp4.Stack(shared.weight[0], shared.scales[0]), chosen,
                                     weights, residual)
    assert_bf16_close(bits_of(got), want, min_exact=0.99)
    direct = ops.moe_down_combine_nvfp4_shared(
        to_device(act), facade.strategy.leaf, facade.strategy.shared,
        torch.from_numpy(chosen[:, :-1].astype(np.int32)).cuda(), torch.from_numpy(weights[:, :-1]).cuda(),
        to_device(residual))
    assert torch.equal(got, direct)


def test_facade_declines_an_uncertified_plane_and_a_missing_shared_leaf():
    from mlx_omnia_amd.kernels.down_combine import DefaultDownCombine, DownCombine, HipNvfp4DownCombine

    _, _, leaf, shared_leaf, *_ = _facade_case(12, 1, 4, paired=False)
    assert isinstance(DownCombine(leaf, hidden=256, inner=512, shared=shared_leaf).strategy, DefaultDownCombine)
    _, _, leaf, _, *_ = _facade_case(13, 1, 4, with_shared=False)
    assert isinstance(DownCombine(leaf, hidden=256, inner=512).strategy, HipNvfp4DownCombine)


def test_shape_checks_raise_before_launch():
    rng = np.random.default_rng(14)
    routed = _leaf(_stack(rng, 4, 32, 512))
    shared = _leaf(_stack(rng, 1, 32, 512))
    act = torch.zeros((2, 5, 512), dtype=torch.bfloat16, device="cuda")
    residual = torch.zeros((2, 32), dtype=torch.bfloat16, device="cuda")
    chosen = torch.zeros((2, 4), dtype=torch.int32, device="cuda")
    weights = torch.zeros((2, 4), dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError):
        ops.moe_down_combine_nvfp4_shared(act, routed, shared, chosen[:, :3].contiguous(), weights, residual)
    with pytest.raises(ValueError):
        ops.moe_down_combine_nvfp4_shared(act, routed, shared, chosen.to(torch.int64), weights, residual)
    with pytest.raises(ValueError):
        ops.moe_down_combine_nvfp4_shared(act[:, :, :256].contiguous(), routed, shared, chosen, weights, residual)
    big = torch.zeros((1, 33, 512), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):   # top_k 32: the kernel takes at most 31 routed slots
        ops.moe_down_combine_nvfp4_shared(big, routed, shared, torch.zeros((1, 32), dtype=torch.int32, device="cuda"),
                                          torch.zeros((1, 32), device="cuda"), residual[:1].contiguous())


def test_golden_fixture():
    golden = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "moe_nvfp4_shared.npz")

    def leaf(name):
        return ops.Nvfp4Leaf(torch.from_numpy(golden[f"{name}_weight"].view(np.int32)).cuda(),
                             torch.from_numpy(golden[f"{name}_scales"]).cuda(), None)

    out = ops.moe_down_combine_nvfp4_shared(
        to_device(golden["act"]), leaf("down"), leaf("shared"), torch.from_numpy(golden["chosen"]).cuda(),
        torch.from_numpy(golden["weights"]).cuda(), to_device(golden["residual"]))
    assert_bf16_close(bits_of(out), golden["out"], min_exact=0.99)

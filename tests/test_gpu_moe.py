"""HIP routed-expert kernels (csrc/moe.hip) against the oracle (oracle/moe.py).

gate_up sums in fp32 in its own order, the oracle rounds the exact dot product once: the
outputs agree bit for bit except where a value sits at a bf16 rounding boundary, so the
bar is at most one bf16 ulp with at least 99% of the outputs identical. down_combine
adds the fp32 SwiGLU, a scaled rounding per expert, the expert sum and the residual: the
north-star bf16 bar (assert_bf16_close) with at least 99% identical.

Shapes: Qwen3-30B-A3B's routed MLP (hidden 2048, inner 768, 128 experts, top-8), an
LFM2-8B-A1B-like one (inner 1792, top-4), ragged sizes that leave lanes idle, 1 to 8
activation vectors per lane in the down kernel (odd and even counts take different
paths), invalid expert ids, k = 1 and k = 16.
"""

import numpy as np
import pytest
import torch

from mlx_omnia_amd.kernels.down_combine import DownCombine, HipDenseDownCombine
from mlx_omnia_amd.kernels.gate_up import GateUp, HipDenseGateUp
from mlx_omnia_amd.kernels.leaf import SwitchLinearLeaf
from mlx_omnia_amd.runtime import ops
from oracle import moe
from oracle.bf16 import from_float, ulp_distance
from util import assert_bf16_close, bits_of, f32_to_device, to_device

pytestmark = pytest.mark.gpu


def _stack(experts, out, inp, seed, scale):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    values = torch.randn((experts, out, inp), generator=gen, device="cuda", dtype=torch.float32)
    return (scale * values).to(torch.bfloat16)


def _gathered(stack, chosen):
    """Host bits of the chosen experts' matrices and the ids remapped onto them (invalid
    ids stay invalid)."""
    experts = stack.shape[0]
    valid = [int(c) for c in chosen if 0 <= c < experts]
    sub = bits_of(stack[torch.tensor(valid, dtype=torch.long, device=stack.device)]) if valid else \
        np.zeros((1, *stack.shape[1:]), dtype=np.uint16)
    remap, slot = [], 0
    for c in chosen:
        if 0 <= c < experts:
            remap.append(slot)
            slot += 1
        else:
            remap.append(-1)
    return sub, np.array(remap, dtype=np.int32)


SHAPES = [
    # experts, hidden, inner, k, seed
    (128, 2048, 768, 8, 1),    # Qwen3-30B-A3B
    (32, 2048, 1792, 4, 2),    # LFM2-8B-A1B-like: 7 vectors per lane in the down kernel
    (8, 520, 72, 3, 3),        # ragged: 65 and 9 vectors per row
    (20, 1024, 256, 1, 4),
    (40, 256, 128, 16, 5),     # sixteen experts: a 16-wave workgroup
    # An even number of vectors per lane in the down kernel (its upper half-wave loads
    # them rotated): 2, 4 with idle lanes, 2 with idle lanes, 8.
    (16, 1024, 512, 8, 6),
    (12, 768, 1000, 6, 7),
    (10, 640, 392, 5, 9),
    (8, 512, 2048, 4, 8),
]


@pytest.mark.parametrize("experts,hidden,inner,k,seed", SHAPES)
def test_gate_up_matches_oracle(experts, hidden, inner, k, seed):
    print(f"moe_gate_up E={experts} H={hidden} I={inner} k={k}", flush=True)
    rng = np.random.default_rng(seed)
    stack = _stack(experts, 2 * inner, hidden, seed, 0.02)
    x = from_float(rng.standard_normal(hidden))
    chosen = rng.choice(experts, size=k, replace=False).astype(np.int32)
    got = bits_of(ops.moe_gate_up(to_device(x), stack, torch.from_numpy(chosen).cuda()))
    sub, remap = _gathered(stack, chosen)
    want = moe.gate_up(x, sub, remap)
    assert got.shape == (k, 2 * inner)
    assert ulp_distance(got, want).max() <= 1
    assert (got == want).mean() >= 0.99


@pytest.mark.parametrize("experts,hidden,inner,k,seed", SHAPES)
def test_down_combine_matches_oracle(experts, hidden, inner, k, seed):
    print(f"moe_down_combine E={experts} H={hidden} I={inner} k={k}", flush=True)
    rng = np.random.default_rng(seed + 100)
    stack = _stack(experts, hidden, inner, seed + 100, 0.03)
    act = from_float(1.5 * rng.standard_normal((k, 2 * inner)))
    chosen = rng.choice(experts, size=k, replace=False).astype(np.int32)
    weights = rng.dirichlet(np.ones(k)).astype(np.float32)
    residual = from_float(rng.standard_normal(hidden))
    got = bits_of(ops.moe_down_combine(to_device(act), stack, torch.from_numpy(chosen).cuda(),
                                       f32_to_device(weights), to_device(residual)))
    sub, remap = _gathered(stack, chosen)
    want = moe.down_combine(act, sub, remap, weights, residual)
    assert got.shape == (hidden,)
    assert_bf16_close(got, want, min_exact=0.99)


def test_invalid_ids_contribute_nothing_and_residual_is_optional():
    experts, hidden, inner = 6, 512, 64
    rng = np.random.default_rng(7)
    gu = _stack(experts, 2 * inner, hidden, 7, 0.05)
    dn = _stack(experts, hidden, inner, 8, 0.05)
    x = from_float(rng.standard_normal(hidden))
    chosen = np.array([2, -1, 6, 5], dtype=np.int32)
    act = ops.moe_gate_up(to_device(x), gu, torch.from_numpy(chosen).cuda())
    act_bits = bits_of(act)
    assert np.all(act_bits[1] == 0) and np.all(act_bits[2] == 0)
    sub, remap = _gathered(gu, chosen)
    assert ulp_distance(act_bits, moe.gate_up(x, sub, remap)).max() <= 1
    weights = np.array([0.4, 0.3, 0.2, 0.1], dtype=np.float32)
    out = bits_of(ops.moe_down_combine(act, dn, torch.from_numpy(chosen).cuda(), f32_to_device(weights)))
    sub, remap = _gathered(dn, chosen)
    assert_bf16_close(out, moe.down_combine(act_bits, sub, remap, weights, None), min_exact=0.99)
    # All routing weights zero: exactly the residual.
    residual = from_float(rng.standard_normal(hidden))
    zero = bits_of(ops.moe_down_combine(act, dn, torch.from_numpy(chosen).cuda(),
                                        f32_to_device(np.zeros(4, np.float32)), to_device(residual)))
    assert np.array_equal(zero, residual)


def test_facades_resolve_to_hip_and_chain():
    experts, hidden, inner, k = 16, 2048, 768, 8
    rng = np.random.default_rng(9)
    gu_leaf = SwitchLinearLeaf(_stack(experts, 2 * inner, hidden, 10, 0.02))
    dn_leaf = SwitchLinearLeaf(_stack(experts, hidden, inner, 11, 0.03))
    gate_up = GateUp(gu_leaf, hidden=hidden, inner=inner, layout="blocked")
    down = DownCombine(dn_leaf, hidden=hidden, inner=inner, layout="blocked")
    assert isinstance(gate_up.strategy, HipDenseGateUp)
    assert isinstance(down.strategy, HipDenseDownCombine)
    # Interleaved layout or a bias: the Core chain serves.
    assert not isinstance(GateUp(gu_leaf, hidden=hidden, inner=inner).strategy, HipDenseGateUp)
    x = from_float(rng.standard_normal(hidden))
    chosen = torch.from_numpy(rng.choice(experts, size=k, replace=False).astype(np.int32)).cuda()
    weights = torch.from_numpy(rng.dirichlet(np.ones(k)).astype(np.float32)).cuda()
    residual = from_float(rng.standard_normal(hidden))
    act = gate_up(to_device(x), chosen)
    out = down(act, chosen, weights, to_device(residual))
    torch.cuda.synchronize()
    ids = chosen.cpu().numpy()
    sub, remap = _gathered(gu_leaf.weight, ids)
    want_act = moe.gate_up(x, sub, remap)
    sub, remap = _gathered(dn_leaf.weight, ids)
    want = moe.down_combine(bits_of(act), sub, remap, weights.cpu().numpy(), residual)
    assert ulp_distance(bits_of(act), want_act).max() <= 1
    assert_bf16_close(bits_of(out), want, min_exact=0.99)


def test_golden_fixture():
    golden = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "moe.npz")
    act = ops.moe_gate_up(to_device(golden["x"]), to_device(golden["gate_up_weight"]),
                          torch.from_numpy(golden["chosen"]).cuda())
    assert ulp_distance(bits_of(act), golden["act"]).max() <= 1
    out = ops.moe_down_combine(to_device(golden["act"]), to_device(golden["down_weight"]),
                               torch.from_numpy(golden["chosen"]).cuda(),
                               f32_to_device(golden["weights"]), to_device(golden["residual"]))
    assert_bf16_close(bits_of(out), golden["out"], min_exact=0.99)

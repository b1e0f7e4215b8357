"""A Qwen3-MoE block step composed from the facades, against the oracle chain.

The facades are declared as the reference's block declares its primitives after load
(models/qwen3/layers/block.py:36-57, models/qwen3/layers/moe.py:34-64), at
Qwen3-30B-A3B's shapes:
- hidden 2048, 32 query heads over 4 kv heads of 128, table rotary (theta = 1e6);
- 128 experts, top-8, expert inner 768, in the blocked gate||up stack the weight
  loader writes.

The step runs `AddRmsNorm` (the join into the layer) -> `QkvRope` (projection, q/k
norm, rotary) -> attention -> o projection -> `ResidualRouter` (the join into the MLP,
its norm, the router, top-8) -> `GateUp` -> `DownCombine` (with the residual), at T = 1
(decode at position 300 over a cache) and T = 512 (prefill). Attention and the two
projections are torch glue: they are not on the path.

Two checks:
- **Stage by stage.** Each primitive's output is checked against the oracle applied to
  the inputs that primitive actually received, to that kernel's own bar. That means: sums,
  logits and indices bit-exact; norms and rotations within the bf16 bar; gate/up within
  one ulp with 99% identical; down/combine within the bf16 bar.
- **End to end.** The oracle chain runs on its own from the block's inputs, the glue
  recomputed by the same torch ops on the oracle's values. Tokens routed alike must
  meet the bf16 bar on the block's output. At least 98% of tokens must route alike;
  at T = 1 the one token must.
"""

import numpy as np
import pytest
import torch

from mlx_omnia_amd.kernels.add_norm import AddRmsNorm, HipAddRmsNorm
from mlx_omnia_amd.kernels.down_combine import DownCombine, HipDenseDownCombine
from mlx_omnia_amd.kernels.gate_up import GateUp, HipDenseGateUp
from mlx_omnia_amd.kernels.leaf import RMSNormLeaf, SwitchLinearLeaf
from mlx_omnia_amd.kernels.qkv_rope import AngleTable, HipQkNormRope, QkvRope, rope_core
from mlx_omnia_amd.kernels.route import HipResidualRouter, ResidualRouter, Routing
from oracle import add_norm, moe, rope, route
from oracle.activations import f64_to_bf16
from oracle.bf16 import from_float, to_f32, ulp_distance
from util import assert_bf16_close, bits_of, to_device

pytestmark = pytest.mark.gpu

H, HQ, HKV, D, PAIRS = 2048, 32, 4, 128, 64
E, K, I = 128, 8, 768
EPS = 1e-6
THETA = 1e6


class Block:
    """Weights (device bf16, seeded) and the facades the reference block declares."""

    def __init__(self, seed: int = 20):
        gen = torch.Generator(device="cuda").manual_seed(seed)

        def w(shape, scale, shift=0.0):
            return (shift + scale * torch.randn(shape, generator=gen, device="cuda")).to(torch.bfloat16)

        self.ln1, self.ln2 = w((H,), 0.1, 1.0), w((H,), 0.1, 1.0)
        self.wqkv = w(((HQ + 2 * HKV) * D, H), H ** -0.5)
        self.qn, self.kn = w((D,), 0.1, 1.0), w((D,), 0.1, 1.0)
        self.wo = w((H, HQ * D), (HQ * D) ** -0.5)
        self.gate = w((E, H), 0.02)
        self.gu = w((E, 2 * I, H), 0.02)
        self.dn = w((E, H, I), 0.03)
        inverse = np.exp(-np.log(THETA) * np.arange(PAIRS) / PAIRS)
        theta = np.arange(4096)[:, None] * inverse[None, :]
        self.cos, self.sin = np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)
        atlas = torch.from_numpy(np.concatenate([self.cos, self.sin], axis=1)).cuda()
        self.table = AngleTable.from_atlas(atlas)

    def declare(self, tokens: int):
        join = AddRmsNorm(RMSNormLeaf(self.ln1, EPS), tokens=1 if tokens == 1 else None)
        prologue = QkvRope(lambda x: x @ self.wqkv.T, heads=HQ, kv_heads=HKV, head_dim=D,
                           rope=lambda x, o: rope_core(x, o, base=THETA), eps=EPS,
                           q_norm=self.qn, k_norm=self.kn, angles=self.table, rotary_pairs=PAIRS)
        router = ResidualRouter(RMSNormLeaf(self.ln2, EPS), self.gate, routing=Routing(experts=E, k=K))
        gate_up = GateUp(SwitchLinearLeaf(self.gu), hidden=H, inner=I, layout="blocked")
        down = DownCombine(SwitchLinearLeaf(self.dn), hidden=H, inner=I, layout="blocked")
        assert isinstance(join.strategy, HipAddRmsNorm)
        assert isinstance(prologue.strategy, HipQkNormRope)
        assert isinstance(router.strategy, HipResidualRouter)
        assert isinstance(gate_up.strategy, HipDenseGateUp)
        assert isinstance(down.strategy, HipDenseDownCombine)
        return join, prologue, router, gate_up, down

    # Glue (torch, on the device): attention over the cache and the o projection.
    def attend(self, q, k, v, cache_k, cache_v):
        """q [1, HQ, T, D], k/v [1, HKV, T, D] for positions P .. P+T-1 after P cached
        rows -> o [T, H] bf16 (causal, fp32 softmax and products)."""
        keys = torch.cat([cache_k, k[0]], dim=1).float()     # [HKV, P+T, D]
        values = torch.cat([cache_v, v[0]], dim=1).float().contiguous()
        length, total = q.shape[2], keys.shape[1]
        group = HQ // HKV
        queries = q[0].float().reshape(HKV, group * length, D).contiguous()
        scores = torch.matmul(queries, keys.transpose(1, 2).contiguous()) * D ** -0.5
        scores = scores.reshape(HKV, group, length, total)
        start = total - length
        mask = torch.arange(total, device="cuda")[None, :] > (start + torch.arange(length, device="cuda"))[:, None]
        probs = torch.softmax(scores.masked_fill(mask, float("-inf")), dim=-1)
        ctx = torch.matmul(probs.reshape(HKV, group * length, total).contiguous(), values)
        ctx = ctx.reshape(HQ, length, D).transpose(0, 1).reshape(length, HQ * D).to(torch.bfloat16)
        return ctx @ self.wo.T


def experts_oracle(h, chosen, weights, residual, gu_host, dn_host):
    """moe.gate_up and moe.down_combine for every token, batched per expert: each
    output is one fp64 dot product of exact products rounded once, as in oracle/moe.py
    (pinned against the per-token oracle on a few tokens below)."""
    tokens = h.shape[0]
    x = to_f32(h).astype(np.float64)
    act = np.zeros((tokens, K, 2 * I), dtype=np.uint16)
    partial = np.zeros((tokens, K, H), dtype=np.float64)
    for e in np.unique(chosen):
        rows, slots = np.nonzero(chosen == e)
        wgu = to_f32(gu_host[e]).astype(np.float64)
        act[rows, slots] = f64_to_bf16(x[rows] @ wgu.T)
        block = to_f32(act[rows, slots])
        a = moe.swiglu_fp32(block[:, :I], block[:, I:]).astype(np.float64)
        partial[rows, slots] = a @ to_f32(dn_host[e]).astype(np.float64).T
    out = np.zeros((tokens, H), dtype=np.uint16)
    for t in range(tokens):
        t32 = partial[t].astype(np.float32)
        d = to_f32(from_float((t32 * weights[t][:, None]).astype(np.float32)))
        total = np.zeros(H, dtype=np.float32)
        for j in range(K):
            total = (total + d[j]).astype(np.float32)
        o = (to_f32(from_float(total)) + to_f32(residual[t])).astype(np.float32)
        out[t] = from_float(o)
    return act, out


def _inputs(tokens, seed):
    rng = np.random.default_rng(seed)
    x = from_float(rng.standard_normal((tokens, H), dtype=np.float32))
    branch = from_float(rng.standard_normal((tokens, H), dtype=np.float32))
    return x, branch


def _cache(position, seed):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    shape = (HKV, position, D)
    return (torch.randn(shape, generator=gen, device="cuda").to(torch.bfloat16),
            torch.randn(shape, generator=gen, device="cuda").to(torch.bfloat16))


@pytest.fixture(scope="module")
def block():
    return Block()


@pytest.mark.parametrize("tokens,position", [(1, 300), (512, 0)])
def test_block_step_stage_by_stage_and_end_to_end(block, tokens, position):
    print(f"qwen3-moe block step tokens={tokens} position={position}", flush=True)
    join, prologue, router, gate_up, down = block.declare(tokens)
    x, branch = _inputs(tokens, seed=tokens + 1)
    cache_k, cache_v = _cache(position, seed=tokens + 2)

    # ---- the block through the facades -------------------------------------------
    resid, n1 = join(to_device(x), to_device(branch))
    q, k, v = prologue(n1[None], position)
    fused = n1[None] @ block.wqkv.T                    # what the prologue projected
    o = block.attend(q, k, v, cache_k, cache_v)
    attended, h, chosen, weights = router(resid, o)
    acts, outs = [], []
    for t in range(tokens):
        act = gate_up(h[t], chosen[t])
        acts.append(act)
        outs.append(down(act, chosen[t], weights[t], attended[t]))
    act_dev, out_dev = torch.stack(acts), torch.stack(outs)
    torch.cuda.synchronize()

    # ---- stage by stage ----------------------------------------------------------
    ln1, ln2, qn, kn = (bits_of(t) for t in (block.ln1, block.ln2, block.qn, block.kn))
    want_s, want_n = add_norm.add_rms_norm(x, branch, ln1, EPS)
    assert np.array_equal(bits_of(resid), want_s)
    assert_bf16_close(bits_of(n1), want_n)

    raw = bits_of(fused[0])
    want_q, want_k = rope.qk_norm_rope(raw[:, : HQ * D].reshape(tokens, HQ, D),
                                       raw[:, HQ * D : (HQ + HKV) * D].reshape(tokens, HKV, D),
                                       qn, kn, block.cos, block.sin, position, EPS, PAIRS)
    assert_bf16_close(bits_of(q[0]), want_q)
    assert_bf16_close(bits_of(k[0]), want_k)
    assert np.array_equal(bits_of(v[0].transpose(0, 1).reshape(tokens, -1)), raw[:, (HQ + HKV) * D :])

    gate = bits_of(block.gate)
    resid_b, o_b = bits_of(resid), bits_of(o)
    want_a, want_h, _, want_idx, want_w = route.residual_rms_router(resid_b, o_b, ln2, gate, EPS, K)
    assert np.array_equal(bits_of(attended), want_a)
    assert_bf16_close(bits_of(h), want_h)
    idx = chosen.cpu().numpy()
    assert np.array_equal(idx, want_idx)
    np.testing.assert_allclose(weights.cpu().numpy(), want_w, rtol=1e-5, atol=1e-7)

    gu_host, dn_host = bits_of(block.gu), bits_of(block.dn)
    h_b, w_np, att_b = bits_of(h), weights.cpu().numpy(), bits_of(attended)
    want_act, _ = experts_oracle(h_b, idx, w_np, att_b, gu_host, dn_host)
    got_act = bits_of(act_dev)
    # The kernel sums in fp32, the oracle rounds the exact sum once. Over 6.3 M outputs,
    # a few cancel to near zero, where a small absolute difference spans many bf16
    # steps. So the bar is the north-star one (absolute, against the largest value),
    # with 99% bit-identical, and one ulp away from cancellation.
    dist = ulp_distance(got_act, want_act)
    big = np.abs(to_f32(want_act)) >= 2.0 ** -6 * np.abs(to_f32(want_act)).max()
    print(f"gate_up: {int((dist > 1).sum())} of {dist.size} beyond one ulp, largest |want| "
          f"among them {np.abs(to_f32(want_act))[dist > 1].max(initial=0.0):.3g}", flush=True)
    assert dist[big].max() <= 1
    assert_bf16_close(got_act, want_act, min_exact=0.99)
    # down/combine from the activation it was given.
    _, want_out = experts_oracle_from_act(got_act, idx, w_np, att_b, dn_host)
    assert_bf16_close(bits_of(out_dev), want_out, min_exact=0.99)
    # The batched restatement equals the per-token oracle on a few tokens.
    for t in sorted({0, tokens // 2, tokens - 1}):
        assert np.array_equal(moe.gate_up(h_b[t], gu_host, idx[t]), want_act[t])
        assert np.array_equal(moe.down_combine(got_act[t], dn_host, idx[t], w_np[t], att_b[t]),
                              want_out[t])

    # ---- end to end: the oracle chain on its own ---------------------------------
    s1, m1 = add_norm.add_rms_norm(x, branch, ln1, EPS)
    fused_o = bits_of(to_device(m1)[None] @ block.wqkv.T)[0]
    q_o, k_o = rope.qk_norm_rope(fused_o[:, : HQ * D].reshape(tokens, HQ, D),
                                 fused_o[:, HQ * D : (HQ + HKV) * D].reshape(tokens, HKV, D),
                                 qn, kn, block.cos, block.sin, position, EPS, PAIRS)
    v_o = to_device(fused_o[:, (HQ + HKV) * D :]).reshape(tokens, HKV, D).transpose(0, 1)[None]
    o_o = bits_of(block.attend(to_device(q_o)[None], to_device(k_o)[None], v_o, cache_k, cache_v))
    a2, h2, _, idx2, w2 = route.residual_rms_router(s1, o_o, ln2, gate, EPS, K)
    _, out2 = experts_oracle(h2, idx2, w2, a2, gu_host, dn_host)
    same = (np.sort(idx2, axis=1) == np.sort(idx, axis=1)).all(axis=1)
    print(f"end to end: {int(same.sum())} of {tokens} tokens routed alike", flush=True)
    assert same.mean() >= (1.0 if tokens == 1 else 0.98)
    assert_bf16_close(bits_of(out_dev)[same], out2[same], min_exact=0.9)


def experts_oracle_from_act(act, chosen, weights, residual, dn_host):
    """moe.down_combine for every token from given activations, batched per expert."""
    tokens = act.shape[0]
    partial = np.zeros((tokens, K, H), dtype=np.float64)
    for e in np.unique(chosen):
        rows, slots = np.nonzero(chosen == e)
        block = to_f32(act[rows, slots])
        a = moe.swiglu_fp32(block[:, :I], block[:, I:]).astype(np.float64)
        partial[rows, slots] = a @ to_f32(dn_host[e]).astype(np.float64).T
    out = np.zeros((tokens, H), dtype=np.uint16)
    for t in range(tokens):
        d = to_f32(from_float((partial[t].astype(np.float32) * weights[t][:, None]).astype(np.float32)))
        total = np.zeros(H, dtype=np.float32)
        for j in range(K):
            total = (total + d[j]).astype(np.float32)
        out[t] = from_float((to_f32(from_float(total)) + to_f32(residual[t])).astype(np.float32))
    return act, out

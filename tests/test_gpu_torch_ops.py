"""`torch.ops.omnia.*` (runtime/torch_ops.py) on the GPU: each operator returns what its
ctypes entry point returns, bit for bit, and a function of several of them traces and
runs under torch.compile (the aot_eager backend, full graph) with the same results."""

import numpy as np
import pytest
import torch

from mlx_omnia_amd.runtime import ops, torch_ops  # noqa: F401  (registers the operators)

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def _bf16(gen, *shape, scale=1.0, shift=0.0):
    return (shift + scale * torch.randn(shape, generator=gen, device="cuda")).to(BF16)


def _same(a, b):
    return a.shape == b.shape and a.dtype == b.dtype and torch.equal(a, b)


def test_each_operator_equals_its_entry_point():
    gen = torch.Generator(device="cuda").manual_seed(0)
    x, r, w = _bf16(gen, 5, 2048), _bf16(gen, 5, 2048), _bf16(gen, 2048, scale=0.1, shift=1.0)
    assert all(_same(a, b) for a, b in zip(torch.ops.omnia.add_rms_norm(x, r, w, 1e-6),
                                           ops.add_rms_norm(x, r, w, 1e-6)))
    raw_q, raw_k = _bf16(gen, 7, 32, 128), _bf16(gen, 7, 8, 128)
    qw, kw = _bf16(gen, 128, scale=0.1, shift=1.0), _bf16(gen, 128, scale=0.1, shift=1.0)
    theta = torch.arange(64, device="cuda")[:, None] * torch.exp(-torch.arange(64, device="cuda") / 64 * 9.2)[None]
    cos, sin = torch.cos(theta).float().contiguous(), torch.sin(theta).float().contiguous()
    got = torch.ops.omnia.qk_norm_rope(raw_q, raw_k, qw, kw, cos, sin, 3, 1e-6, 64, 1.0)
    want = ops.qk_norm_rope(raw_q, raw_k, qw, kw, cos, sin, offset=3, eps=1e-6, rotary_pairs=64)
    assert all(_same(a, b) for a, b in zip(got, want))
    fused = _bf16(gen, 6, 48 * 128)
    got = torch.ops.omnia.rope_epilogue(fused, qw, kw, 32, 8, 128, 11, 19.93, 1e-6)
    want = ops.rope_epilogue(fused, qw, kw, query_heads=32, kv_heads=8, head_dim=128, offset=11, log2_base=19.93,
                             eps=1e-6)
    assert all(_same(a, b) for a, b in zip(got, want))
    tokens = torch.randint(0, 500, (2, 9), generator=gen, device="cuda", dtype=torch.int32)
    table, atlas = _bf16(gen, 500, 256), torch.randn(40, 128, generator=gen, device="cuda")
    got = torch.ops.omnia.embed_atlas(tokens, table, atlas, None, 4, 9)
    want = ops.embed_atlas(tokens, table, atlas, None, position=4, n_positions=9)
    assert _same(got[0], want[0]) and _same(got[1], want[1]) and got[2].numel() == 0
    g, u, a = _bf16(gen, 4, 768), _bf16(gen, 4, 768), _bf16(gen, 4, 32)
    a_log, dt_bias = torch.rand(32, generator=gen, device="cuda") * 2.7, 0.5 * torch.randn(32, generator=gen, device="cuda")
    assert _same(torch.ops.omnia.swiglu(g, u), ops.swiglu(g, u))
    assert _same(torch.ops.omnia.gate_softplus(a, a_log, dt_bias), ops.gate_softplus(a, a_log, dt_bias))
    assert all(_same(p, q) for p, q in zip(torch.ops.omnia.gated_activations(g, u, a, a_log, dt_bias),
                                           ops.gated_activations(g, u, a, a_log, dt_bias)))
    logits, bias = _bf16(gen, 3, 128), 0.1 * torch.randn(128, generator=gen, device="cuda")
    assert all(_same(p, q) for p, q in zip(torch.ops.omnia.softmax_topk(logits, 8), ops.softmax_topk(logits, 8)))
    assert all(_same(p, q) for p, q in zip(torch.ops.omnia.softmax_topk(logits, 8, False, True),
                                           ops.softmax_topk(logits, 8, normalize=False, shared=True)))
    assert all(_same(p, q) for p, q in zip(torch.ops.omnia.sigmoid_topk(logits, bias, 8),
                                           ops.sigmoid_topk(logits, bias, 8)[:2]))
    gate = _bf16(gen, 128, 2048, scale=0.02)
    packed = torch.ops.omnia.pack_router_weight(gate)
    assert _same(packed, ops.pack_router_weight(gate).buffer)
    got = torch.ops.omnia.residual_rms_router(x, r, w, packed, 128, 8, 1e-6)
    want = ops.residual_rms_router(x, r, w, gate, k=8, eps=1e-6)
    assert all(_same(p, q) for p, q in zip(got, (want[0], want[1], want[3], want[4])))


def test_the_steps_either_side_equal_their_entry_points():
    gen = torch.Generator(device="cuda").manual_seed(2)
    x, r = _bf16(gen, 5, 2048), _bf16(gen, 5, 2048)
    w, gate = _bf16(gen, 2048, scale=0.1, shift=1.0), _bf16(gen, 128, 2048, scale=0.02)
    bias = 0.1 * torch.randn(128, generator=gen, device="cuda")
    packed = torch.ops.omnia.pack_router_weight(gate)
    got = torch.ops.omnia.residual_rms_router_sigmoid(x, r, w, packed, bias, 128, 8, 1e-6)
    want = ops.residual_rms_router_sigmoid(x, r, w, gate, bias, k=8, eps=1e-6)
    assert all(_same(p, q) for p, q in zip(got[:3], want[:3]))
    assert _same(got[3].view(torch.int32), want[3].view(torch.int32))
    experts, hidden, inner, k = 16, 2048, 768, 4
    token = _bf16(gen, hidden)
    gate_up, down = _bf16(gen, experts, 2 * inner, hidden, scale=0.02), _bf16(gen, experts, hidden, inner, scale=0.02)
    chosen = torch.tensor([3, 0, 15, 7], dtype=torch.int32, device="cuda")
    weights = torch.tensor([0.4, 0.3, 0.2, 0.1], device="cuda")
    act = torch.ops.omnia.moe_gate_up(token, gate_up, chosen)
    assert _same(act, ops.moe_gate_up(token, gate_up, chosen))
    assert _same(torch.ops.omnia.moe_down_combine(act, down, chosen, weights, token),
                 ops.moe_down_combine(act, down, chosen, weights, token))
    fused, down2 = _bf16(gen, 2 * inner, hidden, scale=0.02), _bf16(gen, hidden, inner, scale=0.02)
    y = torch.ops.omnia.dense_gate_up_swiglu(token, fused)
    assert _same(y, ops.dense_gate_up_swiglu(token, fused))
    assert _same(torch.ops.omnia.dense_down_residual(y, down2, token), ops.dense_down_residual(y, down2, token))
    q, sinks = _bf16(gen, 64, 64), _bf16(gen, 64, scale=2.0)
    cache_k, cache_v = _bf16(gen, 1, 8, 300, 64), _bf16(gen, 1, 8, 300, 64)
    band = torch.arange(300, device="cuda") >= 44
    for mask in (None, band):
        assert _same(torch.ops.omnia.attention_sink_decode(q, cache_k, cache_v, sinks, mask, 0.125),
                     ops.attention_sink_decode(q, cache_k, cache_v, sinks, mask, 0.125))


def test_a_compiled_chain_matches_eager():
    gen = torch.Generator(device="cuda").manual_seed(1)
    x, r, w = _bf16(gen, 4, 2048), _bf16(gen, 4, 2048), _bf16(gen, 2048, scale=0.1, shift=1.0)
    g, u = _bf16(gen, 4, 2048), _bf16(gen, 4, 2048)

    def chain(x, r, w, g, u):
        summed, normed = torch.ops.omnia.add_rms_norm(x, r, w, 1e-6)
        y = torch.ops.omnia.swiglu(g, normed)
        idx, wts = torch.ops.omnia.softmax_topk(y[:, :128].contiguous(), 4)
        return summed, y, idx, wts

    compiled = torch.compile(chain, backend="aot_eager", fullgraph=True)
    eager = chain(x, r, w, g, u)
    for _ in range(2):
        got = compiled(x, r, w, g, u)
        assert all(_same(a, b) for a, b in zip(got, eager))

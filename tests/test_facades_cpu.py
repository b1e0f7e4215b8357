"""Facade resolution, HIP predicates and the Core chains of every primitive, on the CPU.

Mirrors the reference's resolution tests (tests/test_kernel_qk_norm_rope.py,
tests/test_kernel_embedding_rope_atlas.py, tests/test_kernel_moe_route.py,
tests/test_kernel_gate_softplus.py: "a binding binds only where it computes the declared
arithmetic"): on CPU tensors every HIP binding declines or hands the call to its Core
chain, `reference=True` forces the Core chain, and each Core chain agrees with the oracle
on seeded inputs. The HIP kernels themselves are compared with the oracle in
tests/test_gpu_*.py.
"""

import numpy as np
import pytest
import torch

from mlx_omnia_amd.kernels.embed import DefaultEmbed, Embed, applies as embed_applies
from mlx_omnia_amd.kernels.gate_softplus import DefaultGateSoftplus, GateSoftplus
from mlx_omnia_amd.kernels.gate_up import (DefaultGateUpActivation, GateUpActivation, HipSwiGLU,
                                           applies as swiglu_applies)
from mlx_omnia_amd.kernels.leaf import RMSNormLeaf
from mlx_omnia_amd.kernels.qkv_rope import (AngleTable, DefaultQkvRope, QkvRope, qk_norm_rope_applies,
                                            rope_core, rope_epilogue_applies)
from mlx_omnia_amd.kernels.route import (HipSoftmaxTopkRoute, DefaultResidualRouter, DefaultRoute, ResidualRouter, Route,
                                         Routing, residual_router_applies, softmax_topk_applies)
from oracle import activations as act
from oracle import embed as oracle_embed
from oracle import rope as oracle_rope
from oracle import route as oracle_route
from oracle.bf16 import from_float, to_f32, ulp_distance
from util import assert_bf16_close

EPS = 1e-6


def cpu(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


# ---- QK-norm + RoPE ---------------------------------------------------------------


def test_rope_predicates():
    for d, p in ((128, 64), (128, 32), (128, 16), (64, 32), (64, 8), (256, 128), (256, 64)):
        assert qk_norm_rope_applies(d, p), (d, p)
    for d, p in ((128, 48), (96, 48), (128, 128), (64, 4), (128, 0), (512, 256)):
        assert not qk_norm_rope_applies(d, p), (d, p)
    assert rope_epilogue_applies(128) and rope_epilogue_applies(64) and not rope_epilogue_applies(96)


def _qkv_declaration(hq, hkv, d, rng, **extra):
    qw, kw = from_float(1 + 0.1 * rng.standard_normal(d)), from_float(1 + 0.1 * rng.standard_normal(d))
    common = dict(heads=hq, kv_heads=hkv, head_dim=d, rope=lambda x, o: rope_core(x, o, base=1e6),
                  eps=EPS, q_norm=cpu(qw), k_norm=cpu(kw))
    return qw, kw, dict(common, **extra)


def test_qkv_rope_cpu_resolves_to_core_and_matches_epilogue_oracle():
    hq, hkv, d, length, offset = 4, 2, 128, 7, 1234
    rng = np.random.default_rng(0)
    qw, kw, declaration = _qkv_declaration(hq, hkv, d, rng, base=1e6)
    prologue = QkvRope(lambda x: x, **declaration)
    assert isinstance(prologue.strategy, DefaultQkvRope)
    fused = from_float(rng.standard_normal((1, length, (hq + 2 * hkv) * d)))
    q, k, v = prologue(cpu(fused), offset)
    want_q, want_k = oracle_rope.rope_epilogue(fused[0], hq, hkv, d, qw, kw, offset, 1e6, EPS)
    assert_bf16_close(bits(q[0]), want_q)
    assert_bf16_close(bits(k[0]), want_k)
    want_v = fused[0, :, (hq + hkv) * d :].reshape(length, hkv, d).transpose(1, 0, 2)
    assert np.array_equal(bits(v[0]), want_v)


def test_qkv_rope_table_declaration_on_cpu_and_reference_flag():
    rng = np.random.default_rng(1)
    cos, sin = oracle_rope.angle_table(64, 64, 1e6)
    table = AngleTable(torch.from_numpy(cos), torch.from_numpy(sin))
    _, _, declaration = _qkv_declaration(4, 2, 128, rng, angles=table, rotary_pairs=64)
    assert isinstance(QkvRope(lambda x: x, **declaration).strategy, DefaultQkvRope)
    assert isinstance(QkvRope(lambda x: x, reference=True, **declaration).strategy, DefaultQkvRope)


def test_angle_atlas_on_cpu_matches_oracle_and_grows():
    from mlx_omnia_amd.kernels.qkv_rope import AngleAtlas, rope_frequencies
    assert np.array_equal(rope_frequencies(64, 1e6), np.exp(-np.log(1e6) * np.arange(64) / 64))
    atlas = AngleAtlas(64, base=1e6, rows=512)
    cos, sin = oracle_rope.angle_table(2048, 64, 1e6)
    got = atlas.atlas.numpy()
    # torch's and numpy's fp64 cos/sin may differ in a last fp64 bit, which moves an fp32
    # rounding only at a midpoint: one fp32 ulp at most, almost never.
    assert np.abs(got[:, :64] - cos[:512]).max() <= np.spacing(np.float32(1.0))
    assert np.mean(got[:, :64] == cos[:512]) > 0.9999
    kept = atlas.atlas.clone()
    atlas.ensure(1500)
    assert atlas.rows == 1501 and torch.equal(atlas.atlas[:512], kept)
    assert np.abs(atlas.atlas.numpy()[:, 64:] - sin[:1501]).max() <= np.spacing(np.float32(1.0))
    with pytest.raises(ValueError):
        AngleAtlas(64)


def test_angle_atlas_fp32_order_on_cpu_matches_oracle():
    """Laguna's fp32 op order (models/laguna/layers/attention.py:236-243), on the CPU."""
    from mlx_omnia_amd.kernels.qkv_rope import AngleAtlas
    from mlx_omnia_amd.kernels.qkv_rope.atlas import rope_inverse_fp32

    assert np.array_equal(rope_inverse_fp32(64, 1e6), oracle_rope.laguna_inverse(64, 1e6))
    atlas = AngleAtlas(64, base=1e6, rows=300, arithmetic="fp32")
    atlas.ensure(40000)
    cos, sin = oracle_rope.laguna_angle_table(atlas.rows, 64, 1e6)
    got = atlas.atlas.numpy()
    ulp = np.spacing(np.float32(1.0))
    assert np.abs(got[:, :64] - cos).max() <= ulp and np.abs(got[:, 64:] - sin).max() <= ulp
    assert np.mean(got[:, :64] == cos) > 0.9999
    with pytest.raises(ValueError):
        AngleAtlas(64, base=1e6, arithmetic="fp16")


def test_angle_table_contract_and_atlas_view():
    cos, sin = oracle_rope.angle_table(32, 8, 1e4)
    atlas = torch.from_numpy(np.concatenate([cos, sin], axis=-1))
    table = AngleTable.from_atlas(atlas)
    assert table.pairs == 8
    rows = table(5, 3)  # the reference's Angles contract: [length, 2P], cos then sin
    assert rows.shape == (3, 16)
    assert np.array_equal(rows.numpy(), atlas[5:8].numpy())


# ---- Embedding + atlas --------------------------------------------------------------


def test_embed_predicate():
    assert embed_applies(2560, 64, 64, dtype=torch.bfloat16)
    assert embed_applies(256, 32, 0, dtype=torch.bfloat16)
    assert not embed_applies(2562, 64, 64, dtype=torch.bfloat16)
    assert not embed_applies(2560, 62, 64, dtype=torch.bfloat16)
    assert not embed_applies(2560, 64, 64, dtype=torch.float32)
    assert not embed_applies(16384, 64, 64, dtype=torch.bfloat16)


def test_embed_cpu_resolves_to_core_and_matches_oracle():
    rng = np.random.default_rng(2)
    table = from_float(0.02 * rng.standard_normal((100, 64)))
    full = rng.standard_normal((1, 1, 20, 8)).astype(np.float32)
    sliding = rng.standard_normal((1, 1, 20, 16)).astype(np.float32)
    embed = Embed(cpu(table), full_atlas=torch.from_numpy(full), sliding_atlas=torch.from_numpy(sliding))
    assert isinstance(embed.strategy, DefaultEmbed)
    tokens = rng.integers(0, 100, size=(2, 6), dtype=np.int32)
    h, f, s = embed(torch.from_numpy(tokens), 9)
    want_h, want_f, want_s = oracle_embed.embed_atlas(tokens, table, full, sliding, 9, 6)
    assert np.array_equal(bits(h), want_h)
    assert np.array_equal(f.numpy(), want_f) and np.array_equal(s.numpy(), want_s)
    h1, f1, s1 = embed(torch.tensor([[7]], dtype=torch.int32), 3)  # one token: flat rows
    assert h1.shape == (64,) and f1.shape == (8,) and s1.shape == (16,)
    assert np.array_equal(bits(h1), table[7]) and np.array_equal(f1.numpy(), full[0, 0, 3])


# ---- SwiGLU and gate-softplus --------------------------------------------------------


def test_swiglu_binding_declares_only_plain_swiglu():
    assert swiglu_applies(9728) and swiglu_applies(8) and not swiglu_applies(12) and not swiglu_applies(0)
    assert isinstance(GateUpActivation().strategy, HipSwiGLU)
    for kw in (dict(activation="swiglu_oai", limit=7.0), dict(limit=7.0), dict(layout="interleaved")):
        assert isinstance(GateUpActivation(**kw).strategy, DefaultGateUpActivation), kw
    assert isinstance(GateUpActivation(reference=True).strategy, DefaultGateUpActivation)


def test_swiglu_core_chain_on_cpu_tensors_matches_oracle():
    rng = np.random.default_rng(3)
    gate_up = from_float(3 * rng.standard_normal((5, 2 * 48)))
    for activation in (GateUpActivation(), GateUpActivation(reference=True)):
        y = activation(cpu(gate_up))  # CPU tensors: the HIP binding hands over to Core
        want = act.swiglu(gate_up[:, :48], gate_up[:, 48:])
        got = bits(y)
        # torch's CPU sigmoid is not correctly rounded; the oracle's is: a rare one-ulp
        # bf16 difference of the sigmoid may carry through the two products.
        assert ulp_distance(got, want).max() <= 2
        assert (got == want).mean() > 0.98


def test_gate_softplus_cpu_resolves_to_core_and_matches_oracle():
    rng = np.random.default_rng(4)
    a = from_float(4 * rng.standard_normal((9, 32)))
    a_log = rng.uniform(0, 2.7, 32).astype(np.float32)
    dt_bias = (0.5 * rng.standard_normal(32)).astype(np.float32)
    gate = GateSoftplus(torch.from_numpy(a_log), torch.from_numpy(dt_bias))
    assert isinstance(gate.strategy, DefaultGateSoftplus)
    got = gate(cpu(a)).numpy()
    want = act.gate_softplus(a, a_log, dt_bias)
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=0)


def test_gated_activations_pair_on_cpu_resolves_to_core_chains():
    from mlx_omnia_amd.kernels.gated import DefaultGatedActivations, GatedActivations
    from mlx_omnia_amd.runtime.ops import gated_activations_applies

    rng = np.random.default_rng(5)
    gate_up = from_float(3 * rng.standard_normal((6, 2 * 40)))
    a = from_float(4 * rng.standard_normal((6, 32)))
    a_log = rng.uniform(0, 2.7, 32).astype(np.float32)
    dt_bias = (0.5 * rng.standard_normal(32)).astype(np.float32)
    pair = GatedActivations(torch.from_numpy(a_log), torch.from_numpy(dt_bias))
    assert isinstance(pair.strategy, DefaultGatedActivations)  # CPU declaration: Core
    y, g = pair(cpu(gate_up), None, cpu(a))
    want_y = act.swiglu(gate_up[:, :40], gate_up[:, 40:])
    assert ulp_distance(bits(y), want_y).max() <= 2
    np.testing.assert_allclose(g.numpy(), act.gate_softplus(a, a_log, dt_bias), rtol=2e-6, atol=0)
    # The fused kernel's operand conditions beyond the single kernels': even heads, an
    # even row stride of `a`.
    assert gated_activations_applies(cpu(gate_up), cpu(gate_up), cpu(a))
    assert not gated_activations_applies(cpu(gate_up), cpu(gate_up), cpu(a[:, :7]))
    assert not gated_activations_applies(cpu(gate_up), cpu(gate_up), torch.zeros(4, 9)[:, :8])


# ---- Routing ------------------------------------------------------------------------


def test_route_predicates_and_declines():
    assert softmax_topk_applies(128, 8) and softmax_topk_applies(256, 64)
    assert not softmax_topk_applies(257, 8) and not softmax_topk_applies(128, 65)
    assert residual_router_applies(2048, 128, 8) and residual_router_applies(4096, 256, 8)
    assert not residual_router_applies(2560, 128, 8) and not residual_router_applies(2048, 64, 8)
    assert Routing(experts=128, k=8).plain_softmax()
    for knob in (dict(scoring="sigmoid"), dict(bias=torch.zeros(128)), dict(scale=2.5),
                 dict(softcap=30.0), dict(ties="higher"), dict(norm_eps=1e-20)):
        routing = Routing(experts=128, k=8, **knob)
        assert not routing.plain_softmax() and not routing.softmax_slots(), knob
        assert isinstance(Route(None, experts=128, k=8, **knob).strategy, DefaultRoute), knob
    # The shared slot and the unnormalised weights: not the fused router's declaration,
    # but the softmax top-k kernel's (Qwen3.5's shared=True, Qwen3's normalize=norm_topk).
    for knob in (dict(normalize=False), dict(shared=True), dict(normalize=False, shared=True)):
        routing = Routing(experts=128, k=8, **knob)
        assert not routing.plain_softmax() and routing.softmax_slots(), knob
        assert isinstance(Route(None, experts=128, k=8, **knob).strategy, HipSoftmaxTopkRoute), knob
    assert softmax_topk_applies(128, 63, shared=True) and not softmax_topk_applies(128, 64, shared=True)
    assert isinstance(Route(None, experts=128, k=64, shared=True).strategy, DefaultRoute)


def test_route_core_chain_matches_oracle_and_reference_tie_fixture():
    rng = np.random.default_rng(5)
    logits = from_float(rng.standard_normal((50, 128)))
    logits[:6] = from_float(rng.integers(-2, 3, (6, 128)) * 0.5)  # many exact ties
    route = Route(None, experts=128, k=8, reference=True)
    idx, w = route.rows(cpu(logits))
    want_idx, want_w = oracle_route.softmax_topk(logits, 8)
    assert np.array_equal(idx.numpy(), want_idx)
    np.testing.assert_allclose(w.numpy(), want_w, rtol=1e-5, atol=1e-7)
    # The higher-index rule of the reference's softmax chain, on the tie KAT
    # (tests/test_kernel_moe_route.py:152-177): indices 0..7 tie with 11, 35, 67, 99.
    row = np.full((1, 128), from_float(np.array([-1.0]))[0], dtype=np.uint16)
    row[0, [0, 1, 2, 3, 11, 35, 67, 99, 120, 127]] = from_float(np.array([2.0]))[0]
    lower, _ = Route(None, experts=128, k=8, reference=True).rows(cpu(row))
    higher, _ = Route(None, experts=128, k=8, ties="higher").rows(cpu(row))
    assert lower.numpy()[0].tolist() == [0, 1, 2, 3, 11, 35, 67, 99]
    assert higher.numpy()[0].tolist() == [127, 120, 99, 67, 35, 11, 3, 2]


@pytest.mark.parametrize("normalize,shared", [(True, True), (False, False), (False, True)])
def test_route_core_chain_shared_slot_and_unnormalised(normalize, shared):
    """The Core chain's shared slot and unnormalised weights against the oracle; the HIP
    binding, given CPU logits, hands the call to that chain and records it."""
    from mlx_omnia_amd.kernels.resolve import FALLBACKS

    rng = np.random.default_rng(7)
    logits = from_float(rng.standard_normal((40, 128 + shared)) * 2)
    want_idx, want_w = oracle_route.softmax_topk_slots(logits, 8, normalize=normalize, shared=shared)
    core = Route(None, experts=128, k=8, normalize=normalize, shared=shared, reference=True)
    idx, w = core.rows(cpu(logits))
    assert np.array_equal(idx.numpy(), want_idx)
    np.testing.assert_allclose(w.numpy(), want_w, rtol=1e-5, atol=1e-7)
    hip = Route(None, experts=128, k=8, normalize=normalize, shared=shared)
    assert isinstance(hip.strategy, HipSoftmaxTopkRoute)
    name = "HipSoftmaxTopkRoute -> DefaultRoute"
    before = FALLBACKS.get(name, 0)
    idx2, w2 = hip.rows(cpu(logits))
    assert FALLBACKS.get(name, 0) == before + 1
    assert np.array_equal(idx2.numpy(), want_idx)


def test_residual_router_cpu_resolves_to_core_and_matches_oracle():
    rows, hidden, experts, k = 6, 2048, 128, 8
    rng = np.random.default_rng(6)
    x = from_float(rng.standard_normal((rows, hidden)))
    r = from_float(rng.standard_normal((rows, hidden)))
    w = from_float(1 + 0.1 * rng.standard_normal(hidden))
    gate = from_float(0.02 * rng.standard_normal((experts, hidden)))
    router = ResidualRouter(RMSNormLeaf(cpu(w), EPS), cpu(gate), routing=Routing(experts=experts, k=k))
    assert isinstance(router.strategy, DefaultResidualRouter)
    summed, normed, idx, wts = router(cpu(x), cpu(r))
    want = oracle_route.residual_rms_router(x, r, w, gate, EPS, k)
    assert np.array_equal(bits(summed), want[0])
    assert ulp_distance(bits(normed), want[1]).max() <= 1
    # The Core chain's bf16 matmul rounds its fp32 accumulation, the oracle rounds the
    # exact dot product: they agree except for logits at a rounding boundary, so the
    # selections agree wherever the k-th and (k+1)-th logits are apart.
    logits = to_f32(oracle_route.router_logits(want[1], gate))
    for t in range(rows):
        values = np.sort(logits[t])[::-1]
        if values[k - 1] - values[k] < 2.0**-6:  # a near tie at the cut: either pick is fine
            continue
        assert idx.numpy()[t].tolist() == want[3][t].tolist()
    np.testing.assert_allclose(wts.numpy().sum(axis=-1), 1.0, rtol=1e-5)


def test_ordinal_route_predicate_and_core_sigmoid_chain():
    from mlx_omnia_amd.kernels.route import ordinal_keys, ordinal_route_applies, sigmoid_bias_routing
    # ordinal.py:158-174: (experts / 32) * k == 64
    assert ordinal_route_applies(256, 8) and ordinal_route_applies(128, 16) and ordinal_route_applies(1024, 2)
    assert not ordinal_route_applies(128, 8) and not ordinal_route_applies(250, 8)
    bias = torch.zeros(256)
    assert sigmoid_bias_routing(Routing(experts=256, k=8, scoring="sigmoid", bias=bias))
    for knob in (dict(bias=None), dict(scoring="softmax"), dict(normalize=False), dict(scale=2.0),
                 dict(ties="higher"), dict(softcap=10.0)):
        decl = dict(experts=256, k=8, scoring="sigmoid", bias=bias) | knob
        assert not sigmoid_bias_routing(Routing(**decl)), knob
    # On CPU tensors the Core chain serves; it agrees with the oracle off near-ties.
    values = np.random.default_rng(20).standard_normal((20, 256)).astype(np.float32) * 2
    bias = (np.random.default_rng(21).standard_normal(256) * 0.1).astype(np.float32)
    route = Route(None, experts=256, k=8, scoring="sigmoid", bias=torch.from_numpy(bias))
    assert isinstance(route.strategy, DefaultRoute)
    idx, w = route.rows(torch.from_numpy(values))
    want_idx, want_w, want_keys = oracle_route.sigmoid_topk(values, bias, 8)
    assert np.array_equal(idx.numpy(), want_idx)
    np.testing.assert_allclose(w.numpy(), want_w, rtol=1e-6)
    # The Core chain's ordinal keys (ordinal.py:253-262) order the experts as the oracle's.
    scores = torch.sigmoid(torch.from_numpy(values).double()).float()
    keys = ordinal_keys(scores + torch.from_numpy(bias)).numpy()
    assert np.array_equal(keys, want_keys)


def test_call_time_fallback_is_recorded():
    """A built HIP strategy handed logits its kernel does not take passes the call to the
    Core chain and says so (RESOLVED gets the Core module, FALLBACKS counts it)."""
    import importlib

    from mlx_omnia_amd.kernels.route import HipSoftmaxTopkRoute
    resolve = importlib.import_module("mlx_omnia_amd.kernels.resolve")
    routing = Routing(experts=128, k=8)
    strategy = HipSoftmaxTopkRoute(None, routing, DefaultRoute(None, routing))  # built as on a GPU
    resolve.RESOLVED.discard(DefaultRoute.__module__)
    before = resolve.FALLBACKS.get("HipSoftmaxTopkRoute -> DefaultRoute", 0)
    logits = torch.from_numpy(np.random.default_rng(22).standard_normal((4, 128)).astype(np.float32))
    idx, w = strategy.rows(logits)                   # fp32 on the CPU: not the kernel's input
    assert resolve.FALLBACKS["HipSoftmaxTopkRoute -> DefaultRoute"] == before + 1
    assert DefaultRoute.__module__ in resolve.RESOLVED
    want, _ = DefaultRoute(None, routing).rows(logits)
    assert torch.equal(idx, want)


def test_residual_router_core_keys_on_cpu():
    rows, hidden, experts = 3, 2048, 256
    rng = np.random.default_rng(23)
    x = from_float(rng.standard_normal((rows, hidden)))
    r = from_float(rng.standard_normal((rows, hidden)))
    w = from_float(1 + 0.1 * rng.standard_normal(hidden))
    gate = from_float(0.02 * rng.standard_normal((experts, hidden)))
    bias = (rng.standard_normal(experts) * 0.1).astype(np.float32)
    routing = Routing(experts=experts, k=8, scoring="sigmoid", bias=torch.from_numpy(bias))
    router = ResidualRouter(RMSNormLeaf(cpu(w), EPS), cpu(gate), routing=routing)
    assert isinstance(router.strategy, DefaultResidualRouter)
    summed, normed, logits, keys = router.with_keys(cpu(x), cpu(r))
    want = oracle_route.residual_rms_router_sigmoid(x, r, w, gate, bias, EPS, 8)
    assert np.array_equal(bits(summed), want[0])
    # The Core keys order the experts as the Core chain's own logits say.
    core_scores = torch.sigmoid(logits.float()).double() + torch.from_numpy(bias).double()
    order = np.argsort(-core_scores.numpy(), axis=-1, kind="stable")
    assert np.array_equal(np.argsort(keys.numpy().astype(np.int64), axis=-1, kind="stable"), order)


# ---- routed expert gate/up and down/combine ---------------------------------------


def test_moe_predicates():
    from mlx_omnia_amd.kernels.down_combine import dense_down_applies
    from mlx_omnia_amd.kernels.gate_up import dense_gate_up_applies

    for h in (8, 520, 2048, 4096, 8192):
        assert dense_gate_up_applies(h), h
    for h in (0, 4, 100, 8200, 16384):
        assert not dense_gate_up_applies(h), h
    for i in (8, 72, 768, 1792, 2048):
        assert dense_down_applies(i), i
    for i in (0, 12, 2056, 4096):
        assert not dense_down_applies(i), i


def test_moe_cpu_resolves_to_core_and_matches_oracle():
    from mlx_omnia_amd.kernels.down_combine import (DefaultDownCombine, DownCombine,
                                                    HipDenseDownCombine)
    from mlx_omnia_amd.kernels.gate_up import DefaultGateUp, GateUp, HipDenseGateUp
    from mlx_omnia_amd.kernels.leaf import SwitchLinearLeaf
    from oracle import moe as oracle_moe

    experts, hidden, inner = 6, 64, 24
    rng = np.random.default_rng(11)
    gu = from_float(0.05 * rng.standard_normal((experts, 2 * inner, hidden)))
    dn = from_float(0.05 * rng.standard_normal((experts, hidden, inner)))
    x = from_float(rng.standard_normal(hidden))
    chosen = np.array([4, 1, 5], dtype=np.int32)
    weights = np.array([0.5, 0.3, 0.2], dtype=np.float32)
    residual = from_float(rng.standard_normal(hidden))
    gate_up = GateUp(SwitchLinearLeaf(cpu(gu)), hidden=hidden, inner=inner, layout="blocked")
    down = DownCombine(SwitchLinearLeaf(cpu(dn)), hidden=hidden, inner=inner, layout="blocked")
    assert isinstance(gate_up.strategy, DefaultGateUp)
    assert isinstance(down.strategy, DefaultDownCombine)
    assert not isinstance(gate_up.strategy, HipDenseGateUp)
    assert not isinstance(down.strategy, HipDenseDownCombine)
    ids = torch.from_numpy(chosen)
    act = gate_up(cpu(x), ids)
    assert act.shape == (3, 2 * inner)
    # The Core chain's float32 matmul rounds once to bf16 like the oracle's float64 dot.
    assert ulp_distance(bits(act), oracle_moe.gate_up(x, gu, chosen)).max() <= 1
    out = down(act, ids, torch.from_numpy(weights), cpu(residual))
    # The Core chain runs the SwiGLU in bf16 ops (core/kernels/down_combine/default.py:43-58):
    # the dense binding's fp32 activation is the oracle's, so only the north-star bar holds.
    # fp32 routing weights promote the chain's sum to fp32, as mlx promotes it.
    assert out.dtype == torch.float32
    assert_bf16_close(bits(out.to(torch.bfloat16)), oracle_moe.down_combine(bits(act), dn, chosen, weights, residual),
                      min_exact=0.5)
    no_residual = down(act, ids, torch.from_numpy(weights), None)
    assert no_residual.shape == (hidden,)


def test_moe_hip_bindings_decline_other_declarations():
    from mlx_omnia_amd.kernels.down_combine import HipDenseDownCombine
    from mlx_omnia_amd.kernels.gate_up import HipDenseGateUp, OrdinalRouting
    from mlx_omnia_amd.kernels.leaf import SwitchLinearLeaf

    leaf = SwitchLinearLeaf(torch.zeros((4, 48, 64), dtype=torch.bfloat16))
    base = dict(hidden=64, inner=24, activation="silu", limit=None, bias=None, layout="blocked",
                routing=None, shared=None)
    assert HipDenseGateUp.build(leaf, **base) is None  # CPU tensors
    for change in (dict(layout="interleaved"), dict(activation="swiglu_oai"), dict(limit=7.0),
                   dict(routing=OrdinalRouting(2)), dict(bias=torch.zeros(4, 48)),
                   dict(inner=32)):
        assert HipDenseGateUp.build(leaf, **dict(base, **change)) is None, change
    down_leaf = SwitchLinearLeaf(torch.zeros((4, 64, 24), dtype=torch.bfloat16))
    dbase = dict(hidden=64, inner=24, bias=None, shared=None, layout="blocked")
    assert HipDenseDownCombine.build(down_leaf, **dbase) is None
    for change in (dict(layout="interleaved"), dict(bias=torch.zeros(4, 64)), dict(hidden=32)):
        assert HipDenseDownCombine.build(down_leaf, **dict(dbase, **change)) is None, change


@pytest.mark.parametrize("width", (2, 3, 4, 5, 6, 8))
def test_torch_bit_stream_decoder_matches_the_oracle(width):
    from mlx_omnia_amd.kernels.leaf import unpack_words
    from oracle import affine

    rng = np.random.default_rng(width)
    words = rng.integers(0, 1 << 32, size=(3, 5, 4 * width), dtype=np.uint64).astype(np.uint32)
    got = unpack_words(torch.from_numpy(words.view(np.int32)), width)
    assert np.array_equal(got.numpy(), affine.unpack(words, width))


def _affine_leaves(rng, experts, rows, features, bits, group):
    from mlx_omnia_amd.kernels.leaf import QuantizedLinearLeaf, QuantizedSwitchLinearLeaf
    from oracle import affine

    words = rng.integers(0, 1 << 32, size=(experts, rows, features * bits // 32), dtype=np.uint64)
    words = words.astype(np.uint32)
    scale = 4.0 / ((1 << bits) * np.sqrt(features))
    s = from_float(scale * (0.5 + rng.random((experts, rows, features // group))))
    b = from_float(-to_f32(s) * ((1 << bits) - 1) / 2)
    stack = affine.Stack(words, s, b, group, bits)
    leaf = QuantizedSwitchLinearLeaf(torch.from_numpy(words.view(np.int32)), cpu(s), cpu(b), group, bits)
    single = QuantizedLinearLeaf(leaf.weight[0], leaf.scales[0], leaf.biases[0], group, bits)
    return stack, leaf, single


@pytest.mark.parametrize("width", (3, 4, 8))
def test_affine_moe_cpu_resolves_to_core_and_matches_oracle(width):
    from mlx_omnia_amd.kernels.down_combine import DefaultDownCombine, DownCombine, HipAffineDownCombine
    from mlx_omnia_amd.kernels.gate_up import DefaultGateUp, GateUp, HipAffineGateUp
    from oracle import affine

    experts, hidden, inner = 5, 128, 64
    rng = np.random.default_rng(width)
    gstack, gleaf, _ = _affine_leaves(rng, experts, 2 * inner, hidden, width, 32)
    dstack, dleaf, _ = _affine_leaves(rng, experts, hidden, inner, width, 64)
    gate_up = GateUp(gleaf, hidden=hidden, inner=inner)
    down = DownCombine(dleaf, hidden=hidden, inner=inner)
    assert isinstance(gate_up.strategy, DefaultGateUp) and isinstance(down.strategy, DefaultDownCombine)
    assert HipAffineGateUp.build(gleaf, hidden=hidden, inner=inner, activation="silu", limit=None,
                                 bias=None, layout="interleaved", routing=None, shared=None) is None
    assert HipAffineDownCombine.build(dleaf, hidden=hidden, inner=inner, bias=None, shared=None,
                                      layout="interleaved") is None
    x = from_float(rng.standard_normal(hidden))
    chosen = np.array([4, 0, 2], dtype=np.int32)
    act_core = gate_up(cpu(x), torch.from_numpy(chosen))
    # The Core chain's sigmoid is torch's, its dot an fp32 sum: one ulp from the oracle.
    want_act = affine.gate_up(x, gstack, chosen)
    assert ulp_distance(bits(act_core), want_act).max() <= 1
    weights = to_f32(from_float(np.array([0.5, 0.3, 0.2])))
    residual = from_float(rng.standard_normal(hidden))
    out = down(act_core, torch.from_numpy(chosen), torch.from_numpy(weights).to(torch.bfloat16),
               cpu(residual))
    # The Core chain rounds the weighted rows and their sum at other points than the kernel.
    assert_bf16_close(bits(out), affine.down_combine(bits(act_core), dstack, chosen, weights, residual),
                      min_exact=0.8)


def test_affine_core_chain_serves_the_shared_slot_and_the_clamp():
    from mlx_omnia_amd.kernels.gate_up import GateUp
    from oracle import affine

    experts, hidden, inner = 4, 64, 32
    rng = np.random.default_rng(12)
    gstack, gleaf, _ = _affine_leaves(rng, experts, 2 * inner, hidden, 4, 32)
    sstack, _, shared = _affine_leaves(rng, 1, 2 * inner, hidden, 2, 64)
    x = from_float(2 * rng.standard_normal(hidden))
    gate_up = GateUp(gleaf, hidden=hidden, inner=inner, limit=0.5, shared=shared)
    got = gate_up(cpu(x), torch.tensor([3, 1, 7], dtype=torch.int32))
    want = affine.gate_up(x, gstack, [3, 1, 7], limit=0.5,
                          shared=affine.Stack(sstack.weight[0], sstack.scales[0], sstack.biases[0], 64, 2))
    assert ulp_distance(bits(got), want).max() <= 1


def test_affine_bindings_decline_other_declarations():
    from mlx_omnia_amd.kernels.down_combine import affine_down_applies
    from mlx_omnia_amd.kernels.gate_up import affine_gate_up_applies

    assert affine_gate_up_applies(2048, 64, 4) and affine_gate_up_applies(96, 32, 3)
    for args in ((2048, 16, 4), (2048, 64, 7), (1000, 32, 4), (2048 + 64, 128, 4), (32768, 32, 4)):
        assert not affine_gate_up_applies(*args), args
    assert affine_down_applies(768, 64, 4) and affine_down_applies(1536, 128, 8)
    for args in ((2048, 64, 4), (768, 48, 4), (100, 32, 2), (768, 64, 1)):
        assert not affine_down_applies(*args), args


def test_ordinal_routing_keeps_the_best_keys_lowest_index_first():
    from mlx_omnia_amd.kernels.gate_up import OrdinalRouting

    keys = torch.tensor([5, 2, 9, 2, 0, 7], dtype=torch.int32)
    assert OrdinalRouting(3).indices(keys).tolist() == [4, 1, 3]


# ---- dense SwiGLU MLP ---------------------------------------------------------------


def test_mlp_predicates():
    from mlx_omnia_amd.kernels.mlp import dense_down_residual_applies, dense_gate_up_swiglu_applies

    assert dense_gate_up_swiglu_applies(2560, 9728) and dense_gate_up_swiglu_applies(8192, 8)
    assert not dense_gate_up_swiglu_applies(8200, 64) and not dense_gate_up_swiglu_applies(100, 64)
    assert dense_down_residual_applies(2560, 9728) and dense_down_residual_applies(16, 25600)
    assert not dense_down_residual_applies(2560, 100)


def test_mlp_cpu_resolves_to_core_and_matches_oracle():
    from mlx_omnia_amd.kernels.leaf import SwiGLU
    from mlx_omnia_amd.kernels.mlp import DefaultMlp, HipDenseMlp, Mlp
    from oracle import mlp as oracle_mlp

    hidden, inner = 128, 256
    rng = np.random.default_rng(12)
    fused = from_float(0.1 * rng.standard_normal((2 * inner, hidden)))
    down = from_float(0.05 * rng.standard_normal((hidden, inner)))
    leaf = SwiGLU(hidden, inner).to(torch.bfloat16)
    with torch.no_grad():
        leaf.gate_up_proj.weight.copy_(cpu(fused))
        leaf.down_proj.weight.copy_(cpu(down))
    mlp = Mlp(leaf, hidden=hidden, inner=inner)
    assert isinstance(mlp.strategy, DefaultMlp)
    assert HipDenseMlp.build(leaf, hidden=hidden, inner=inner, activation="silu") is None  # CPU
    assert isinstance(Mlp(leaf, hidden=hidden, inner=inner, activation="gelu_tanh").strategy, DefaultMlp)
    x = from_float(rng.standard_normal(hidden))
    residual = from_float(rng.standard_normal(hidden))
    with torch.no_grad():
        out = mlp(cpu(x), cpu(residual))
    # The Core chain rounds at the op boundaries of torch's bf16 ops (silu in one op, not
    # the kernel's bf16 steps): the same MLP, not the same bits (the reference's own
    # facade test, tests/test_kernel_dense_mlp.py:104-122, bounds it at 2^-5).
    want = to_f32(oracle_mlp.mlp(x, fused, down, residual))
    got = out.float().numpy()
    assert np.abs(got - want).max() / np.abs(want).max() < 2.0**-5


def test_mlp_hip_binding_declines_other_leaves():
    from mlx_omnia_amd.kernels.leaf import SwiGLU
    from mlx_omnia_amd.kernels.mlp import HipDenseMlp

    leaf = SwiGLU(64, 32)  # fp32 weights
    assert HipDenseMlp.build(leaf, hidden=64, inner=32, activation="silu") is None
    leaf = leaf.to(torch.bfloat16)
    assert HipDenseMlp.build(leaf, hidden=64, inner=32, activation="gelu_tanh") is None
    assert HipDenseMlp.build(leaf, hidden=64, inner=16, activation="silu") is None  # shape

    class Quantized(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.gate_up_proj = torch.nn.Identity()
            self.down_proj = torch.nn.Identity()

    assert HipDenseMlp.build(Quantized(), hidden=64, inner=32, activation="silu") is None


# ---- decode attention step ----------------------------------------------------------


def test_attention_predicates_and_declines():
    from mlx_omnia_amd.kernels.attention import (AttentionStep, DefaultAttentionStep, FixedKVCache,
                                                 HipAttentionStep, attention_step_applies)
    from mlx_omnia_amd.kernels.qkv_rope import AngleTable

    assert attention_step_applies(32, 8, 128, 64) and attention_step_applies(16, 16, 128, 8)
    assert not attention_step_applies(32, 8, 64, 32)      # head_dim
    assert not attention_step_applies(48, 3, 128, 64)     # gqa 16
    assert not attention_step_applies(32, 8, 128, 4)      # pairs
    assert not attention_step_applies(30, 8, 128, 64)     # not grouped evenly
    cache = FixedKVCache.empty(2, 16, 128)
    table = AngleTable.from_atlas(torch.zeros(64, 128))
    weight = torch.ones(128, dtype=torch.bfloat16)
    common = dict(heads=8, kv_heads=2, head_dim=128, scale=0.1, dtype=torch.bfloat16,
                  query_weight=weight, key_weight=weight, eps=1e-6, rotary_pairs=64, mscale=1.0,
                  angles=table, base=0.0, sinks=None)
    assert HipAttentionStep.build(cache, **common) is None           # CPU tensors
    assert HipAttentionStep.build(cache, **dict(common, sinks=torch.zeros(8))) is None
    assert HipAttentionStep.build(cache, **dict(common, angles=None)) is None
    assert HipAttentionStep.build(cache, **dict(common, query_weight=None)) is None
    assert isinstance(AttentionStep(cache, **{k: v for k, v in common.items()}).strategy,
                      DefaultAttentionStep)


def test_captured_step_refuses_replays_past_the_angle_table():
    """A capture over a ring cache needs the last position its replays reach, covered by
    the table; a fixed cache needs the table to cover its capacity."""
    from mlx_omnia_amd.kernels.attention import FixedKVCache, RingKVCache, capture_covered

    fixed = FixedKVCache.empty(2, 64, 128)
    capture_covered(fixed, 64)
    with pytest.raises(ValueError, match="covering the cache's 64 rows"):
        capture_covered(fixed, 63)
    ring = RingKVCache.empty(2, 16, 128)
    ring.offset = 40
    with pytest.raises(ValueError, match="prepare_capture"):
        capture_covered(ring, 4096)                  # no bound declared
    ring.replay_limit = 39
    with pytest.raises(ValueError, match="prepare_capture"):
        capture_covered(ring, 4096)                  # a bound behind the position
    ring.replay_limit = 100
    capture_covered(ring, 101)
    with pytest.raises(ValueError, match="past the angle table's 100 rows"):
        capture_covered(ring, 100)


def test_attention_core_chain_matches_oracle_on_cpu():
    from mlx_omnia_amd.kernels.attention import AttentionStep, FixedKVCache, RingKVCache
    from mlx_omnia_amd.kernels.qkv_rope import AngleTable
    from oracle import attention as attn
    from oracle.rope import angle_table

    heads, kv_heads, pairs, d = 8, 2, 32, 128
    rng = np.random.default_rng(13)
    cos, sin = angle_table(64, pairs, 10000.0)
    atlas = np.concatenate([cos, sin], axis=1)
    table = AngleTable.from_atlas(torch.from_numpy(atlas))
    qw = from_float(1 + 0.1 * rng.standard_normal(d))
    kw = from_float(1 + 0.1 * rng.standard_normal(d))
    for cache, window in ((FixedKVCache.empty(kv_heads, 24, d), 0), (RingKVCache.empty(kv_heads, 8, d), 8)):
        step = AttentionStep(cache, heads=heads, kv_heads=kv_heads, head_dim=d, scale=d ** -0.5,
                             dtype=torch.bfloat16, query_weight=cpu(qw), key_weight=cpu(kw),
                             rotary_pairs=pairs, angles=table)
        rows = cache.keys.shape[2]
        keys = np.zeros((kv_heads, rows, d), np.uint16)
        values = np.zeros_like(keys)
        for position in range(12):
            q, k, v = (from_float(rng.standard_normal(n * d)) for n in (heads, kv_heads, kv_heads))
            got = bits(step(*(cpu(x).reshape(1, 1, -1) for x in (q, k, v))).reshape(heads, d))
            want, keys, values = attn.decode_step(q, k, v, qw, kw, atlas[position], keys, values,
                                                  position, window=window, scale=d ** -0.5,
                                                  eps=1e-6, pairs=pairs)
            # The chain's norm sums in fp32 (the oracle in fp64) and its softmax is torch's:
            # the same step at the north-star bar.
            assert_bf16_close(got, want, min_exact=0.9)
            keys, values = bits(cache.keys[0]), bits(cache.values[0])
        assert cache.offset == 12


def test_torch_mxfp4_decoder_matches_the_oracle():
    from mlx_omnia_amd.kernels.leaf import mxfp4_dequantize
    from oracle import mxfp4

    rng = np.random.default_rng(31)
    words = rng.integers(0, 1 << 32, size=(3, 5, 16), dtype=np.uint64).astype(np.uint32)
    scales = rng.integers(0, 200, size=(3, 5, 4)).astype(np.uint8)
    scales[0, 0, :2] = (0, 1)                 # a zero factor and the smallest normal one
    got = mxfp4_dequantize(torch.from_numpy(words.view(np.int32)), torch.from_numpy(scales))
    want = mxfp4.dequantize(mxfp4.Stack(words, scales, None))
    assert np.array_equal(got.numpy().astype(np.float64), want)


def _mxfp4_leaf(rng, experts, rows, features):
    from mlx_omnia_amd.kernels.leaf import QuantizedSwitchLinearLeaf
    from oracle import mxfp4

    words = rng.integers(0, 1 << 32, size=(experts, rows, features // 8), dtype=np.uint64).astype(np.uint32)
    scales = rng.integers(119, 123, size=(experts, rows, features // 32)).astype(np.uint8)
    b = from_float(0.25 * rng.standard_normal((experts, rows)))
    leaf = QuantizedSwitchLinearLeaf(torch.from_numpy(words.view(np.int32)), torch.from_numpy(scales),
                                     None, 32, 4, mode="mxfp4")
    return mxfp4.Stack(words, scales, b), leaf, cpu(b)


def test_mxfp4_moe_cpu_resolves_to_core_and_matches_oracle():
    from mlx_omnia_amd.kernels.down_combine import DefaultDownCombine, DownCombine, HipMxfp4DownCombine
    from mlx_omnia_amd.kernels.gate_up import DefaultGateUp, GateUp, HipMxfp4GateUp
    from oracle import mxfp4

    experts, hidden, inner = 6, 128, 64
    rng = np.random.default_rng(32)
    gstack, gleaf, gbias = _mxfp4_leaf(rng, experts, 2 * inner, hidden)
    dstack, dleaf, dbias = _mxfp4_leaf(rng, experts, hidden, inner)
    declared = dict(hidden=hidden, inner=inner, activation="swiglu_oai", limit=7.0, bias=gbias)
    gate_up = GateUp(gleaf, **declared)
    down = DownCombine(dleaf, hidden=hidden, inner=inner, bias=dbias)
    assert isinstance(gate_up.strategy, DefaultGateUp) and isinstance(down.strategy, DefaultDownCombine)
    assert HipMxfp4GateUp.build(gleaf, layout="interleaved", routing=None, shared=None, **declared) is None
    assert HipMxfp4DownCombine.build(dleaf, hidden=hidden, inner=inner, bias=dbias, shared=None,
                                     layout="interleaved") is None
    x = from_float(2 * rng.standard_normal(hidden))
    chosen = np.array([5, 0, 3, 1], dtype=np.int32)
    act_core = gate_up(cpu(x), torch.from_numpy(chosen))
    # The Core chain rounds 1.702 g to bf16 before the sigmoid: the same function, looser.
    np.testing.assert_allclose(to_f32(bits(act_core)), to_f32(mxfp4.gate_up(x, gstack, chosen, 7.0)),
                               rtol=0.06, atol=0.02)
    weights = to_f32(from_float(rng.dirichlet(np.ones(4))))
    residual = from_float(rng.standard_normal(hidden))
    out = down(act_core, torch.from_numpy(chosen), torch.from_numpy(weights).to(torch.bfloat16),
               cpu(residual))
    # The Core chain rounds the row before the bias add and sums in bf16.
    assert_bf16_close(bits(out), mxfp4.down_combine(bits(act_core), dstack, chosen, weights, residual),
                      min_exact=0.8)


def test_mxfp4_predicate():
    from mlx_omnia_amd.kernels.gate_up import mxfp4_applies

    assert mxfp4_applies(2880, 2880) and mxfp4_applies(32, 32)
    for args in ((2880, 2888), (2888, 2880), (0, 32), (32, 0)):
        assert not mxfp4_applies(*args), args


def test_torch_nvfp4_decoder_matches_the_oracle():
    from mlx_omnia_amd.kernels.leaf import nvfp4_dequantize
    from oracle import nvfp4

    rng = np.random.default_rng(33)
    words = rng.integers(0, 1 << 32, size=(3, 5, 16), dtype=np.uint64).astype(np.uint32)
    scales = rng.integers(0, 256, size=(3, 5, 8)).astype(np.uint8)
    scales[0, 0, :4] = (0x7F, 0xFF, 0x01, 0x80)
    got = nvfp4_dequantize(torch.from_numpy(words.view(np.int32)), torch.from_numpy(scales))
    assert np.array_equal(got.numpy().astype(np.float64), nvfp4.dequantize(nvfp4.Stack(words, scales)))


def test_nvfp4_moe_cpu_resolves_to_core_and_matches_oracle():
    from mlx_omnia_amd.kernels.down_combine import DefaultDownCombine, DownCombine, HipNvfp4DownCombine
    from mlx_omnia_amd.kernels.gate_up import DefaultGateUp, GateUp, HipNvfp4GateUp
    from mlx_omnia_amd.kernels.leaf import QuantizedSwitchLinearLeaf
    from oracle import nvfp4

    experts, hidden, inner = 5, 128, 64
    rng = np.random.default_rng(34)

    def leaf(rows, features):
        words = rng.integers(0, 1 << 32, size=(experts, rows, features // 8), dtype=np.uint64).astype(np.uint32)
        scales = rng.integers(0x18, 0x28, size=(experts, rows, features // 16)).astype(np.uint8)
        return nvfp4.Stack(words, scales), QuantizedSwitchLinearLeaf(
            torch.from_numpy(words.view(np.int32)), torch.from_numpy(scales), None, 16, 4, mode="nvfp4")

    gstack, gleaf = leaf(2 * inner, hidden)
    dstack, dleaf = leaf(hidden, inner)
    gate_up = GateUp(gleaf, hidden=hidden, inner=inner)
    down = DownCombine(dleaf, hidden=hidden, inner=inner)
    assert isinstance(gate_up.strategy, DefaultGateUp) and isinstance(down.strategy, DefaultDownCombine)
    assert HipNvfp4GateUp.build(gleaf, hidden=hidden, inner=inner, activation="silu", limit=None, bias=None,
                                layout="interleaved", routing=None, shared=None) is None
    assert HipNvfp4DownCombine.build(dleaf, hidden=hidden, inner=inner, bias=None, shared=None,
                                     layout="interleaved") is None
    x = from_float(2 * rng.standard_normal(hidden))
    chosen = np.array([4, 0, 2], dtype=np.int32)
    act_core = gate_up(cpu(x), torch.from_numpy(chosen))
    # The Core chain's sigmoid and product are bf16 tensor ops: one ulp from the oracle.
    assert ulp_distance(bits(act_core), nvfp4.gate_up(x, gstack, chosen)).max() <= 1
    weights = to_f32(from_float(np.array([0.5, 0.3, 0.2])))
    residual = from_float(rng.standard_normal(hidden))
    out = down(act_core, torch.from_numpy(chosen), torch.from_numpy(weights).to(torch.bfloat16), cpu(residual))
    assert_bf16_close(bits(out), nvfp4.down_combine(bits(act_core), dstack, chosen, weights, residual),
                      min_exact=0.8)


def test_nvfp4_ordinal_routing_core_chain_matches_a_stable_argsort():
    from mlx_omnia_amd.kernels.gate_up import DefaultGateUp, GateUp, HipNvfp4GateUp, OrdinalRouting
    from mlx_omnia_amd.kernels.leaf import QuantizedSwitchLinearLeaf
    from oracle import nvfp4

    experts, hidden, inner = 40, 64, 32
    rng = np.random.default_rng(35)
    words = rng.integers(0, 1 << 32, size=(experts, 2 * inner, hidden // 8), dtype=np.uint64).astype(np.uint32)
    scales = rng.integers(0x18, 0x28, size=(experts, 2 * inner, hidden // 16)).astype(np.uint8)
    leaf = QuantizedSwitchLinearLeaf(torch.from_numpy(words.view(np.int32)), torch.from_numpy(scales), None, 16, 4,
                                     mode="nvfp4")
    gate_up = GateUp(leaf, hidden=hidden, inner=inner, routing=OrdinalRouting(top_k=5))
    assert isinstance(gate_up.strategy, DefaultGateUp)      # CPU tensors: the Core chain
    assert HipNvfp4GateUp.build(leaf, hidden=hidden, inner=inner, activation="silu", limit=None, bias=None,
                                layout="interleaved", routing=OrdinalRouting(top_k=5), shared=None) is None
    keys = rng.integers(0, 1 << 32, size=experts, dtype=np.uint64).astype(np.uint32)
    keys[[7, 11, 30]] = keys[2]                              # ties resolve to the lower index
    x = from_float(rng.standard_normal(hidden))
    got = gate_up(cpu(x), torch.from_numpy(keys))
    chosen = list(np.argsort(keys.astype(np.uint64), kind="stable")[:5])
    assert ulp_distance(bits(got), nvfp4.gate_up(x, nvfp4.Stack(words, scales), chosen)).max() <= 1


def test_packed_nvfp4_certificate_agrees_with_the_oracle_and_cpu_declines():
    """The facade's certificate of the halved plane (kernels/down_combine) against the
    oracle's restatement of shared/nvfp4/packed.py:126-164, and the packed binding's
    shape rule (nvfp4_packed.py:185-190); on CPU tensors the declaration reaches Core."""
    from mlx_omnia_amd.kernels.down_combine import (DefaultDownCombine, DownCombine, packed_down_applies,
                                                    packed_plane_certified)
    from mlx_omnia_amd.kernels.leaf import QuantizedLinearLeaf, QuantizedSwitchLinearLeaf
    from oracle import nvfp4

    rng = np.random.default_rng(40)
    base = rng.integers(0, 0x7F, size=(3, 16, 32)).astype(np.uint8)
    base[..., 1::2] = base[..., 0::2]
    planes = [base]
    first = base.copy()
    first[0, 0, 1] ^= 0x11
    planes.append(first)
    other = base.copy()
    other[2, 5, 7] ^= 0x01
    planes.append(other)
    signed = base.copy()
    signed[1, 3, 4:6] = 0x85
    planes.append(signed)
    for plane in planes:
        want = nvfp4.halved_scales(plane) is not None
        assert packed_plane_certified(torch.from_numpy(plane)) == want
    assert [packed_plane_certified(torch.from_numpy(p)) for p in planes] == [True, True, False, False]

    assert packed_down_applies(64, 512, 4) and packed_down_applies(2048, 512, 31)
    assert not packed_down_applies(64, 256, 4) and not packed_down_applies(66, 512, 4)
    assert not packed_down_applies(64, 512, 32) and not packed_down_applies(64, 512, 0)

    words = torch.from_numpy(rng.integers(0, 1 << 32, size=(3, 64, 64), dtype=np.uint64).astype(np.uint32).view(np.int32))
    scales = torch.from_numpy(np.repeat(base[:, :, ::2], 2, axis=-1)[:, :4].repeat(16, axis=1)[:, :64])
    leaf = QuantizedSwitchLinearLeaf(words, scales[..., :32], None, 16, 4, mode="nvfp4")
    shared = QuantizedLinearLeaf(words[0], scales[0, :, :32], None, 16, 4, mode="nvfp4")
    facade = DownCombine(leaf, hidden=64, inner=512, shared=shared)
    assert isinstance(facade.strategy, DefaultDownCombine)


def test_sink_attention_core_chain_matches_the_oracle_on_a_growing_cache():
    """The Core chain with sinks over `KVCache` (no norms, no rotation, so the queries are
    the raw rows): a causal prefill, then a decode step under a boolean band, each query
    against oracle.attention.sink_attend over the rows it may see; on CPU tensors the
    HIP sink binding declines."""
    from mlx_omnia_amd.kernels.attention import AttentionStep, DefaultAttentionStep, KVCache
    from oracle import attention as oracle_attention

    rng = np.random.default_rng(50)
    heads, kv_heads, length = 8, 2, 6
    sinks = from_float(2.0 * rng.standard_normal(heads))
    cache = KVCache()
    step = AttentionStep(cache, heads=heads, kv_heads=kv_heads, head_dim=64, scale=0.125, dtype=torch.bfloat16,
                         sinks=torch.from_numpy(to_f32(sinks)).to(torch.bfloat16))
    assert isinstance(step.strategy, DefaultAttentionStep)

    def raw(t, count):
        return torch.from_numpy(rng.standard_normal((1, t, count * 64))).to(torch.bfloat16)

    def bits(t):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)

    q, k, v = raw(length, heads), raw(length, kv_heads), raw(length, kv_heads)
    out = step(q, k, v, mask="causal")
    assert cache.offset == length and cache.capacity == KVCache.BLOCK
    keys, values = bits(cache.keys[0, :, :length]), bits(cache.values[0, :, :length])
    for i in range(length):
        want = oracle_attention.sink_attend(bits(q[0, i].reshape(heads, 64)), keys, values, sinks,
                                            np.arange(length) <= i, 0.125)
        assert_bf16_close(bits(out[0, :, i]), want, min_exact=0.95)
    q, k, v = raw(1, heads), raw(1, kv_heads), raw(1, kv_heads)
    band = torch.arange(length + 1) >= 3
    out = step(q, k, v, mask=band)
    keys, values = bits(cache.keys[0, :, : length + 1]), bits(cache.values[0, :, : length + 1])
    want = oracle_attention.sink_attend(bits(q[0, 0].reshape(heads, 64)), keys, values, sinks, band.numpy(), 0.125)
    assert_bf16_close(bits(out[0, :, 0]), want, min_exact=0.95)

"""The weight-layout rules (mlx-omnia_amd/checkpoint.py) on a synthetic sharded
checkpoint: every fused tensor is checked element-for-element against the source leaves
it was built from (byte moves: bit-exact), the sources leave the dict, and the facades
built on the fused tensors compute what the unfused projections compute.

The layouts are those the reference's loader builds (mlx_omnia/engine/checkpoint.py:
277-451, models/lfm2/moe/checkpoint.py:43-60); the checks follow its loader tests' names
and shapes.
"""

import numpy as np
import pytest
import torch

from checkpoint_fixture import EXPERTS, HEAD_DIM, HEADS, HIDDEN, INNER, KV_HEADS, MOE_INNER, make
from mlx_omnia_amd import checkpoint as ckpt

L = ckpt.LAYOUTS


@pytest.fixture()
def loaded(tmp_path):
    source = make(tmp_path / "ckpt")
    return source, ckpt.read_checkpoint(tmp_path / "ckpt")


def _eq(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_load_shards_merges_every_shard(loaded, tmp_path):
    source, weights = loaded
    assert sorted(weights) == sorted(source)
    assert all(_eq(weights[k], source[k]) for k in source)
    with pytest.raises(FileNotFoundError):
        ckpt.read_checkpoint(tmp_path / "missing")


def test_fuse_qkv_concatenates_weights_and_biases(loaded):
    source, weights = loaded
    weights = ckpt.apply(weights, L["qkv"])
    for layer in range(2):
        a = f"model.layers.{layer}.self_attn."
        fused = weights[f"{a}qkv_proj.weight"]
        q, k, v = (source[f"{a}{n}_proj.weight"] for n in "qkv")
        assert fused.shape == ((HEADS + 2 * KV_HEADS) * HEAD_DIM, HIDDEN) and fused.is_contiguous()
        assert _eq(fused[: q.shape[0]], q) and _eq(fused[q.shape[0] : q.shape[0] + k.shape[0]], k)
        assert _eq(fused[q.shape[0] + k.shape[0] :], v)
        bias = weights[f"{a}qkv_proj.bias"]
        assert _eq(bias, torch.cat([source[f"{a}{n}_proj.bias"] for n in "qkv"]))
        assert not any(f"{a}{n}_proj.weight" in weights for n in "qkv")


def test_fuse_qkv_moves_mixed_formats_instead_of_fusing(loaded):
    source, weights = loaded
    a = "model.layers.0.self_attn."
    weights[f"{a}k_proj.weight"] = weights[f"{a}k_proj.weight"].float()
    weights = ckpt.apply(weights, L["qkv"])
    assert f"{a}qkv_proj.weight" not in weights
    assert _eq(weights[f"{a}qkv_proj.q_proj.weight"], source[f"{a}q_proj.weight"])
    assert weights[f"{a}qkv_proj.k_proj.weight"].dtype == torch.float32
    assert ckpt.leaf_format(weights, {"weight": f"{a}qkv_proj.q_proj.weight"}) != ckpt.leaf_format(
        weights, {"weight": f"{a}qkv_proj.k_proj.weight"})


def test_concat_gate_up_puts_gate_rows_first(loaded):
    source, weights = loaded
    weights = ckpt.apply(weights, L["dense_gate_up"])
    fused = weights["model.layers.0.mlp.gate_up_proj.weight"]
    assert fused.shape == (2 * INNER, HIDDEN)
    assert _eq(fused[:INNER], source["model.layers.0.mlp.gate_proj.weight"])
    assert _eq(fused[INNER:], source["model.layers.0.mlp.up_proj.weight"])
    assert "model.layers.0.mlp.gate_proj.weight" not in weights


def test_stack_and_block_experts(loaded):
    source, weights = loaded
    weights = ckpt.apply(weights, L["moe_blocked"])
    w13 = weights["model.layers.1.mlp.switch_mlp.gate_up_proj.weight"]
    w2 = weights["model.layers.1.mlp.switch_mlp.down_proj.weight"]
    assert w13.shape == (EXPERTS, 2 * MOE_INNER, HIDDEN) and w2.shape == (EXPERTS, HIDDEN, MOE_INNER)
    for e in range(EXPERTS):
        x = f"model.layers.1.mlp.experts.{e}."
        assert _eq(w13[e, :MOE_INNER], source[f"{x}gate_proj.weight"])
        assert _eq(w13[e, MOE_INNER:], source[f"{x}up_proj.weight"])
        assert _eq(w2[e], source[f"{x}down_proj.weight"])
    assert not any(".experts." in key for key in weights)


def test_interleave_gate_up_alternates_rows(loaded):
    source, weights = loaded
    weights = ckpt.apply(weights, L["moe_interleaved"])
    fused = weights["model.layers.1.mlp.switch_mlp.gate_up_proj.weight"]
    for e in range(EXPERTS):
        x = f"model.layers.1.mlp.experts.{e}."
        assert _eq(fused[e, 0::2], source[f"{x}gate_proj.weight"])
        assert _eq(fused[e, 1::2], source[f"{x}up_proj.weight"])


def test_split_stacked_gate_up_transposes_halves():
    gen = torch.Generator().manual_seed(1)
    fused = torch.randn(3, HIDDEN, 2 * MOE_INNER, generator=gen).to(torch.bfloat16)
    down = torch.randn(3, MOE_INNER, HIDDEN, generator=gen).to(torch.bfloat16)
    weights = {"model.layers.0.mlp.experts.gate_up_proj": fused,
               "model.layers.0.mlp.experts.down_proj": down}
    weights = ckpt.apply(weights, L["moe_halves"][:1])
    t = "model.layers.0.mlp.switch_mlp."
    assert _eq(weights[f"{t}gate_proj.weight"], fused[..., :MOE_INNER].transpose(-2, -1))
    assert _eq(weights[f"{t}up_proj.weight"], fused[..., MOE_INNER:].transpose(-2, -1))
    assert _eq(weights[f"{t}down_proj.weight"], down.transpose(-2, -1))


def test_norm_folding_tied_head_and_casts(loaded):
    source, weights = loaded
    folded = ckpt.apply(dict(weights), L["fold_norms"])
    assert torch.equal(folded["model.norm.weight"], source["model.norm.weight"] + 1)
    assert torch.equal(folded["model.layers.0.self_attn.q_norm.weight"],
                       source["model.layers.0.self_attn.q_norm.weight"] + 1)
    assert torch.equal(folded["model.layers.0.mlp.gate_proj.weight"], source["model.layers.0.mlp.gate_proj.weight"])
    prepared = ckpt.prepare(dict(weights), L["qkv"], dtype=torch.float32, tie_word_embeddings=True)
    assert "lm_head.weight" not in prepared
    assert prepared["model.layers.0.self_attn.qkv_proj.weight"].dtype == torch.float32
    with pytest.raises(ValueError, match="quantised"):
        ckpt.prepare({"a.scales": torch.zeros(1)}, (), dtype=torch.float16)


def test_stack_refuses_an_incomplete_expert_set(loaded):
    _, weights = loaded
    del weights["model.layers.1.mlp.experts.2.up_proj.weight"]
    with pytest.raises(ValueError, match="missing for experts"):
        ckpt.apply(weights, L["moe_blocked"])


def test_scopes_match_whole_module_components(loaded):
    """The dense gate||up rule (scope `mlp`) leaves `switch_mlp` alone, and a layout runs
    on every layer it finds without being told the layer count."""
    source, weights = loaded
    weights = ckpt.apply(weights, (ckpt.Stack("mlp"),) + L["dense_gate_up"])
    assert "model.layers.1.mlp.switch_mlp.gate_up_proj.weight" not in weights
    assert weights["model.layers.1.mlp.switch_mlp.gate_proj.weight"].shape == (EXPERTS, MOE_INNER, HIDDEN)
    assert weights["model.layers.0.mlp.gate_up_proj.weight"].shape == (2 * INNER, HIDDEN)


def test_quantised_leaves_fuse_every_suffix():
    """A quantised leaf's scales and biases ride along with its packed words."""
    gen = torch.Generator().manual_seed(4)
    weights = {}
    a = "model.layers.0.self_attn."
    for name, rows in (("q", 8), ("k", 4), ("v", 4)):
        weights[f"{a}{name}_proj.weight"] = torch.randint(0, 1 << 30, (rows, 6), generator=gen, dtype=torch.int32)
        weights[f"{a}{name}_proj.scales"] = torch.randn(rows, 3, generator=gen).to(torch.bfloat16)
        weights[f"{a}{name}_proj.biases"] = torch.randn(rows, 3, generator=gen).to(torch.bfloat16)
    source = dict(weights)
    ckpt.apply(weights, L["qkv"])
    assert sorted(weights) == [f"{a}qkv_proj.{s}" for s in ("biases", "scales", "weight")]
    for suffix in ("weight", "scales", "biases"):
        assert torch.equal(weights[f"{a}qkv_proj.{suffix}"],
                           torch.cat([source[f"{a}{n}_proj.{suffix}"] for n in "qkv"]))


def test_fused_layouts_drive_the_facades(loaded):
    """The dense MLP and the routed expert pair built on the fused tensors compute what
    the separate projections compute (the Core chains on the CPU)."""
    from mlx_omnia_amd.kernels.down_combine import DownCombine
    from mlx_omnia_amd.kernels.gate_up import GateUp
    from mlx_omnia_amd.kernels.leaf import SwiGLU, SwitchLinearLeaf
    from mlx_omnia_amd.kernels.mlp import Mlp

    source, weights = loaded
    weights = ckpt.apply(weights, L["dense_gate_up"] + L["moe_blocked"])
    gen = torch.Generator().manual_seed(2)
    x = torch.randn(HIDDEN, generator=gen).to(torch.bfloat16)
    residual = torch.randn(HIDDEN, generator=gen).to(torch.bfloat16)

    leaf = SwiGLU(HIDDEN, INNER).to(torch.bfloat16)
    with torch.no_grad():
        leaf.gate_up_proj.weight.copy_(weights["model.layers.0.mlp.gate_up_proj.weight"])
        leaf.down_proj.weight.copy_(weights["model.layers.0.mlp.down_proj.weight"])
        got = Mlp(leaf, hidden=HIDDEN, inner=INNER)(x, residual)
    m = "model.layers.0.mlp."
    g = source[f"{m}gate_proj.weight"].float() @ x.float()
    u = source[f"{m}up_proj.weight"].float() @ x.float()
    want = source[f"{m}down_proj.weight"].float() @ (g * torch.sigmoid(g) * u) + residual.float()
    np.testing.assert_allclose(got.float().numpy(), want.numpy(), rtol=3e-2, atol=3e-2)

    chosen = torch.tensor([3, 1], dtype=torch.int32)
    route_w = torch.tensor([0.7, 0.3])
    gate_up = GateUp(SwitchLinearLeaf(weights["model.layers.1.mlp.switch_mlp.gate_up_proj.weight"]),
                     hidden=HIDDEN, inner=MOE_INNER, layout="blocked")
    down = DownCombine(SwitchLinearLeaf(weights["model.layers.1.mlp.switch_mlp.down_proj.weight"]),
                       hidden=HIDDEN, inner=MOE_INNER, layout="blocked")
    out = down(gate_up(x, chosen), chosen, route_w, residual).float()
    want = residual.float().clone()
    for e, w in zip(chosen.tolist(), route_w.tolist()):
        xx = f"model.layers.1.mlp.experts.{e}."
        g = source[f"{xx}gate_proj.weight"].float() @ x.float()
        u = source[f"{xx}up_proj.weight"].float() @ x.float()
        want += w * (source[f"{xx}down_proj.weight"].float() @ (g * torch.sigmoid(g) * u))
    np.testing.assert_allclose(out.numpy(), want.numpy(), rtol=3e-2, atol=3e-2)

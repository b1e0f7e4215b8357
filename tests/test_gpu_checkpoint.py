"""A checkpoint loaded straight onto the GPU, fused there, drives the HIP kernels: the
dense MLP (`omnia_dense_gate_up_swiglu`, `omnia_dense_down_residual`) and the routed
expert pair (`omnia_moe_gate_up`, `omnia_moe_down_combine`) on the fused tensors match
the oracle fed with layouts built independently in numpy from the source leaves."""

import numpy as np
import pytest
import torch

from checkpoint_fixture import EXPERTS, HIDDEN, INNER, MOE_INNER, make
from mlx_omnia_amd import checkpoint as ckpt
from mlx_omnia_amd.kernels.down_combine import DownCombine, HipDenseDownCombine
from mlx_omnia_amd.kernels.gate_up import GateUp, HipDenseGateUp
from mlx_omnia_amd.kernels.leaf import SwiGLU, SwitchLinearLeaf
from mlx_omnia_amd.kernels.mlp import HipDenseMlp, Mlp
from oracle import mlp as oracle_mlp
from oracle import moe as oracle_moe
from oracle.bf16 import from_float
from util import assert_bf16_close, bits_of, f32_to_device, to_device

pytestmark = pytest.mark.gpu


def test_device_load_fuse_and_run(tmp_path):
    print("checkpoint: load to cuda, fuse, run dense MLP and routed experts", flush=True)
    source = {k: bits_of(v) for k, v in make(tmp_path / "ckpt").items()}
    weights = ckpt.read_checkpoint(tmp_path / "ckpt", device="cuda")
    assert all(t.device.type == "cuda" for t in weights.values())
    layouts = ckpt.LAYOUTS
    weights = ckpt.apply(weights, layouts["qkv"] + layouts["dense_gate_up"] + layouts["moe_blocked"])
    fused = weights["model.layers.0.mlp.gate_up_proj.weight"]
    assert fused.is_contiguous() and fused.data_ptr() % 16 == 0

    rng = np.random.default_rng(3)
    x = from_float(rng.standard_normal(HIDDEN))
    residual = from_float(rng.standard_normal(HIDDEN))

    leaf = SwiGLU(HIDDEN, INNER).to(device="cuda", dtype=torch.bfloat16)
    with torch.no_grad():
        leaf.gate_up_proj.weight.copy_(fused)
        leaf.down_proj.weight.copy_(weights["model.layers.0.mlp.down_proj.weight"])
    mlp = Mlp(leaf, hidden=HIDDEN, inner=INNER)
    assert isinstance(mlp.strategy, HipDenseMlp)
    with torch.no_grad():
        got = bits_of(mlp(to_device(x), to_device(residual)))
    m = "model.layers.0.mlp."
    fused_np = np.concatenate([source[f"{m}gate_proj.weight"], source[f"{m}up_proj.weight"]])
    want = oracle_mlp.mlp(x, fused_np, source[f"{m}down_proj.weight"], residual)
    assert_bf16_close(got, want, min_exact=0.95)

    w13 = weights["model.layers.1.mlp.switch_mlp.gate_up_proj.weight"]
    w2 = weights["model.layers.1.mlp.switch_mlp.down_proj.weight"]
    gate_up = GateUp(SwitchLinearLeaf(w13), hidden=HIDDEN, inner=MOE_INNER, layout="blocked")
    down = DownCombine(SwitchLinearLeaf(w2), hidden=HIDDEN, inner=MOE_INNER, layout="blocked")
    assert isinstance(gate_up.strategy, HipDenseGateUp) and isinstance(down.strategy, HipDenseDownCombine)
    chosen = np.array([2, 0, 3], dtype=np.int32)
    route_w = np.array([0.5, 0.3, 0.2], dtype=np.float32)
    ids = torch.from_numpy(chosen).cuda()
    act = gate_up(to_device(x), ids)
    out = bits_of(down(act, ids, f32_to_device(route_w), to_device(residual)))
    e = "model.layers.1.mlp.experts."
    stack13 = np.stack([np.concatenate([source[f"{e}{i}.gate_proj.weight"], source[f"{e}{i}.up_proj.weight"]])
                        for i in range(EXPERTS)])
    stack2 = np.stack([source[f"{e}{i}.down_proj.weight"] for i in range(EXPERTS)])
    want_act = oracle_moe.gate_up(x, stack13, chosen)
    assert_bf16_close(bits_of(act), want_act, min_exact=0.95)
    assert_bf16_close(out, oracle_moe.down_combine(bits_of(act), stack2, chosen, route_w, residual), min_exact=0.95)

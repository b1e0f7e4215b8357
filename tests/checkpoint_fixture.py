"""A small synthetic checkpoint in the HuggingFace layout, written with safetensors.

Two layers: layer 0 a dense trunk (q/k/v with a bias, gate/up/down), layer 1 a routed
MLP with per-expert leaves; norms, an embedding and a tied lm_head; split over two
shards. Values are seeded normals rounded to bf16.
"""

from __future__ import annotations

from pathlib import Path

import torch

HIDDEN, INNER, EXPERTS, MOE_INNER, HEADS, KV_HEADS, HEAD_DIM = 64, 96, 4, 32, 4, 2, 16


def make(directory: Path, seed: int = 0) -> dict[str, torch.Tensor]:
    from safetensors.torch import save_file

    gen = torch.Generator().manual_seed(seed)

    def t(*shape, scale=0.1):
        return (scale * torch.randn(*shape, generator=gen)).to(torch.bfloat16)

    tensors: dict[str, torch.Tensor] = {"model.embed_tokens.weight": t(100, HIDDEN),
                                        "lm_head.weight": t(100, HIDDEN),
                                        "model.norm.weight": t(HIDDEN)}
    for layer in range(2):
        a = f"model.layers.{layer}.self_attn."
        tensors[f"{a}q_proj.weight"] = t(HEADS * HEAD_DIM, HIDDEN)
        tensors[f"{a}k_proj.weight"] = t(KV_HEADS * HEAD_DIM, HIDDEN)
        tensors[f"{a}v_proj.weight"] = t(KV_HEADS * HEAD_DIM, HIDDEN)
        tensors[f"{a}q_proj.bias"] = t(HEADS * HEAD_DIM)
        tensors[f"{a}k_proj.bias"] = t(KV_HEADS * HEAD_DIM)
        tensors[f"{a}v_proj.bias"] = t(KV_HEADS * HEAD_DIM)
        tensors[f"{a}q_norm.weight"] = t(HEAD_DIM)
        tensors[f"model.layers.{layer}.input_layernorm.weight"] = t(HIDDEN)
    m = "model.layers.0.mlp."
    tensors[f"{m}gate_proj.weight"] = t(INNER, HIDDEN)
    tensors[f"{m}up_proj.weight"] = t(INNER, HIDDEN)
    tensors[f"{m}down_proj.weight"] = t(HIDDEN, INNER)
    for e in range(EXPERTS):
        x = f"model.layers.1.mlp.experts.{e}."
        tensors[f"{x}gate_proj.weight"] = t(MOE_INNER, HIDDEN)
        tensors[f"{x}up_proj.weight"] = t(MOE_INNER, HIDDEN)
        tensors[f"{x}down_proj.weight"] = t(HIDDEN, MOE_INNER)
    names = sorted(tensors)
    half = len(names) // 2
    directory.mkdir(parents=True, exist_ok=True)
    save_file({k: tensors[k] for k in names[:half]}, str(directory / "model-00001-of-00002.safetensors"))
    save_file({k: tensors[k] for k in names[half:]}, str(directory / "model-00002-of-00002.safetensors"))
    return tensors

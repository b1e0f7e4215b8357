"""Weight layouts for the fused kernels, built from safetensors checkpoints.

The dict side of the reference's loader (mlx_omnia/engine/checkpoint.py:277-444, and the
LFM2 expert stacking in models/lfm2/moe/checkpoint.py:43-60), over torch tensors: the
fusions take a flat `{name: tensor}` dict and return it with the projections the kernels
read fused, the sources removed so that only one copy stays resident.

- `fuse_qkv` (checkpoint.py:303-330): q/k/v concatenated on the output axis for every
  suffix they carry (weight, bias, and a quantised leaf's scales/biases); leaves of
  different formats move under `qkv_proj.{q,k,v}_proj.*` instead of into one matrix.
- `concat_gate_up` (:333-347): a dense trunk's gate and up concatenated, gate rows first,
  the `SwiGLU` leaf's `gate_up_proj` (what `omnia_dense_gate_up_swiglu` reads).
- `stack_experts` (:350-373): per-expert leaves stacked into `[experts, out, in]` under
  `switch_mlp.*`, the `SwitchLinear` layout.
- `block_gate_up`: each expert's gate and up concatenated on the output axis,
  `[experts, 2 * inner, in]`, the "blocked" layout `omnia_moe_gate_up` reads (LFM2's `w13`,
  models/lfm2/moe/checkpoint.py:43-60); `interleave_gate_up` (:410-426) builds the row
  interleave the Core chain's `SwitchGLU` reads.
- `split_stacked_gate_up` (:376-394), `fold_norm_scales` (:397-407), `drop_tied_head`
  (:440-444), `reject_dtype_cast` (:446-451) and `prepare_weights` (:617-636) as there.

`load_shards` reads every `model*.safetensors` of a directory with safetensors' own
loader (it executes nothing from the file), straight onto `device` when one is given:
on an MI355X the fusions then run on the GPU and the fused tensors are born contiguous
and 16-byte aligned, ready for the kernels. Each fusion frees its sources as it goes, so
the peak stays near one extra layer's worth of memory.
"""

from __future__ import annotations

from pathlib import Path
from typing import Callable, Iterable, Mapping, Sequence

import torch

QKV = ("q", "k", "v")
QKV_SUFFIXES = ("weight", "scales", "biases", "bias")
FORMAT_SUFFIXES = ("weight", "scales", "biases")

Weights = dict[str, torch.Tensor]
Fusion = Callable[[Weights], Weights]

__all__ = [
    "block_gate_up", "concat_gate_up", "drop_tied_head", "fold_norm_scales", "fusible",
    "fuse_qkv", "interleave_gate_up", "load_shards", "prepare_weights", "reject_dtype_cast",
    "split_stacked_gate_up", "stack_experts",
]


def load_shards(directory: Path | str, device: torch.device | str | None = None) -> Weights:
    """Every `model*.safetensors` shard of `directory`, merged (the index file only says
    which shard holds what)."""
    from safetensors.torch import load_file

    weights: Weights = {}
    shards = sorted(Path(directory).glob("model*.safetensors"))
    if not shards:
        raise FileNotFoundError(f"no model*.safetensors under {directory}")
    target = "cpu" if device is None else str(device)
    for shard in shards:
        weights.update(load_file(str(shard), device=target))
    return weights


def fusible(weights: Mapping[str, torch.Tensor], keys: Sequence[str]) -> bool:
    """Whether leaves sharing an input carry one format, read off the tensors: the same
    trailing shape and dtype for all of them, or none of them present."""
    present = [key for key in keys if key in weights]
    if not present:
        return True
    if len(present) != len(keys):
        return False
    return len({(tuple(weights[key].shape[1:]), weights[key].dtype) for key in present}) == 1


def _cat(parts: Iterable[torch.Tensor], dim: int = 0) -> torch.Tensor:
    return torch.cat(list(parts), dim=dim).contiguous()


def fuse_qkv(weights: Weights, layers: int) -> Weights:
    for layer in range(layers):
        prefix = f"model.layers.{layer}.self_attn."
        if not all(f"{prefix}{name}_proj.weight" in weights for name in QKV):
            continue
        same = all(fusible(weights, [f"{prefix}{name}_proj.{suffix}" for name in QKV])
                   for suffix in QKV_SUFFIXES)
        if not same:
            for name in QKV:
                for suffix in QKV_SUFFIXES:
                    key = f"{prefix}{name}_proj.{suffix}"
                    if key in weights:
                        weights[f"{prefix}qkv_proj.{name}_proj.{suffix}"] = weights.pop(key)
            continue
        for suffix in QKV_SUFFIXES:
            keys = [f"{prefix}{name}_proj.{suffix}" for name in QKV]
            if all(key in weights for key in keys):
                weights[f"{prefix}qkv_proj.{suffix}"] = _cat(weights.pop(key) for key in keys)
    return weights


def concat_gate_up(weights: Weights, layers: int, *, prefix: str = "mlp") -> Weights:
    for layer in range(layers):
        leaf = f"model.layers.{layer}.{prefix}."
        for suffix in FORMAT_SUFFIXES:
            keys = [f"{leaf}{name}_proj.{suffix}" for name in ("gate", "up")]
            if all(key in weights for key in keys):
                weights[f"{leaf}gate_up_proj.{suffix}"] = _cat(weights.pop(key) for key in keys)
    return weights


def stack_experts(weights: Weights, layers: int, experts: int, *, prefix: str = "mlp") -> Weights:
    for layer in range(layers):
        source = f"model.layers.{layer}.{prefix}.experts."
        target = f"model.layers.{layer}.{prefix}.switch_mlp."
        for name in ("gate_proj", "up_proj", "down_proj"):
            for suffix in FORMAT_SUFFIXES:
                if f"{source}0.{name}.{suffix}" not in weights:
                    continue
                parts = [weights.pop(f"{source}{expert}.{name}.{suffix}") for expert in range(experts)]
                weights[f"{target}{name}.{suffix}"] = torch.stack(parts).contiguous()
                del parts
    return weights


def block_gate_up(weights: Weights, layers: int, *, prefix: str = "mlp") -> Weights:
    """`switch_mlp.{gate,up}_proj` [E, inner, in] -> `switch_mlp.gate_up_proj`
    [E, 2 * inner, in]: each expert's gate rows, then its up rows."""
    for layer in range(layers):
        leaf = f"model.layers.{layer}.{prefix}.switch_mlp."
        for suffix in FORMAT_SUFFIXES:
            keys = [f"{leaf}{name}_proj.{suffix}" for name in ("gate", "up")]
            if all(key in weights for key in keys):
                weights[f"{leaf}gate_up_proj.{suffix}"] = _cat((weights.pop(key) for key in keys), dim=1)
    return weights


def interleave_gate_up(weights: Weights, layers: int, *, prefix: str = "mlp") -> Weights:
    """[E, inner, in] gate and up -> [E, 2 * inner, in] rows g0, u0, g1, u1, ..."""
    for layer in range(layers):
        leaf = f"model.layers.{layer}.{prefix}.switch_mlp."
        for suffix in FORMAT_SUFFIXES:
            keys = [f"{leaf}{name}_proj.{suffix}" for name in ("gate", "up")]
            if not all(key in weights for key in keys):
                continue
            parts = [weights.pop(key) for key in keys]
            experts, rows, cols = parts[0].shape
            weights[f"{leaf}gate_up_proj.{suffix}"] = torch.stack(parts, dim=2).reshape(
                experts, 2 * rows, cols).contiguous()
    return weights


def split_stacked_gate_up(weights: Weights, layers: int) -> Weights:
    """`experts.gate_up_proj` [E, in, 2 * inner] (gate and up in halves) and
    `experts.down_proj` [E, inner, in] -> `switch_mlp.*` in the [E, out, in] layout."""
    for layer in range(layers):
        source = f"model.layers.{layer}.mlp.experts."
        target = f"model.layers.{layer}.mlp.switch_mlp."
        fused = weights.pop(f"{source}gate_up_proj", None)
        if fused is None:
            continue
        middle = fused.shape[-1] // 2
        weights[f"{target}gate_proj.weight"] = fused[..., :middle].transpose(-2, -1).contiguous()
        weights[f"{target}up_proj.weight"] = fused[..., middle:].transpose(-2, -1).contiguous()
        del fused
        weights[f"{target}down_proj.weight"] = weights.pop(f"{source}down_proj").transpose(-2, -1).contiguous()
    return weights


def fold_norm_scales(weights: Weights) -> Weights:
    """Norm weights stored centred on zero (`scale = 1 + w`) folded to plain gains."""
    for key, value in weights.items():
        if key.endswith(("layernorm.weight", "q_norm.weight", "k_norm.weight")) or key == "model.norm.weight":
            weights[key] = value + 1
    return weights


def drop_tied_head(weights: Weights) -> None:
    """Tied checkpoints still serialise lm_head; it is dropped."""
    for suffix in FORMAT_SUFFIXES:
        weights.pop(f"lm_head.{suffix}", None)


def reject_dtype_cast(dtype: torch.dtype | None, weights: Mapping[str, torch.Tensor]) -> None:
    """A quantised checkpoint (it carries `.scales`) cannot be cast to a float dtype."""
    if dtype is not None and any(key.endswith(".scales") for key in weights):
        raise ValueError("dtype= cannot be applied to a quantized checkpoint")


def prepare_weights(weights: Weights, fusions: Sequence[Fusion], *, dtype: torch.dtype | None = None,
                    tie_word_embeddings: bool = False) -> Weights:
    """Reject a cast over packed tensors, cast, drop the tied head, fuse in order."""
    reject_dtype_cast(dtype, weights)
    if dtype is not None:
        weights = {key: value.to(dtype) for key, value in weights.items()}
    if tie_word_embeddings:
        drop_tied_head(weights)
    for fuse in fusions:
        weights = fuse(weights)
    return weights

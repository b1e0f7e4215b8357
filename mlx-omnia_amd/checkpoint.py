"""Weight layouts the fused kernels read, built from a checkpoint's flat tensor dict.

A layout is a tuple of declarative rules over the checkpoint's key space, and one
engine (`apply`) runs them. Every key is parsed into (module, leaf, suffix):
`model.layers.3.self_attn.q_proj.weight` is module `model.layers.3.self_attn`, leaf
`q_proj`, suffix `weight` (a quantised leaf adds `scales` and `biases` suffixes). The
rules:

- `Join`: in every module whose path ends with `scope`, the `parts` leaves become one
  leaf `into`, each suffix arranged as the kernel reads it: "rows" (stacked on the output
  axis: q, k, v for `omnia_qk_norm_rope`'s fused projection, gate then up for
  `omnia_dense_gate_up_swiglu`), "blocked" (per expert, gate rows then up rows on axis 1:
  `omnia_moe_gate_up`'s layout) or "interleaved" (per expert, gate and up rows
  alternating: the Core `SwitchGLU` order). Parts whose formats differ (a format being
  the set of suffixes with their dtypes and trailing shapes) are nested under
  `into.part` instead, as separate leaves;
- `Stack`: per-expert modules `<owner>.experts.<i>` become one module
  `<owner>.<into>` whose leaves are stacked over the expert index ([experts, out, in],
  the `SwitchLinear` layout); the expert count is read off the keys;
- `Halves`: a stacked [experts, in, 2 * inner] leaf stored without suffix (gate and up
  as halves of the last axis) becomes two [experts, inner, in] leaves, and its partner
  down leaf [experts, inner, in] the transposed [experts, in, inner];
- `Shift` adds a constant to the matching keys (norm gains stored centred on zero);
  `Drop` removes them (a tied head serialised anyway).

`prepare` casts (refused for a quantised checkpoint, whose packed words cannot be
cast), drops a tied head, then applies a layout. `LAYOUTS` names the layout each kernel
family reads. Every rule removes its sources as it builds its target, so only one copy
of each weight stays resident.

The layouts, key names and the cases handled are those of the reference's loader
(mlx_omnia/engine/checkpoint.py:277-451 and 617-636: q/k/v fusion with the mixed-format
fallback, gate||up concatenation, expert stacking, stacked gate_up halves, norm
folding, tied heads, the quantised-cast refusal) and of LFM2's blocked `w13`
(models/lfm2/moe/checkpoint.py:43-60).

`read_checkpoint` reads every `model*.safetensors` shard of a directory with
safetensors' own loader (it executes nothing from the file), straight onto `device`
when one is given: the rules then run on the GPU and every fused tensor is born
contiguous and 16-byte aligned, as the kernels require.
"""

from __future__ import annotations

import re
from collections import defaultdict
from dataclasses import dataclass
from pathlib import Path
from typing import Literal, Mapping, Protocol, Sequence

import torch

Weights = dict[str, torch.Tensor]
Arrangement = Literal["rows", "blocked", "interleaved"]

__all__ = [
    "Drop", "Halves", "Join", "LAYOUTS", "Shift", "Stack", "apply", "leaf_format", "prepare",
    "read_checkpoint",
]


class Rule(Protocol):
    def __call__(self, weights: Weights) -> None: ...


def _parse(key: str) -> tuple[str, str, str]:
    """(module, leaf, suffix) of a dotted key; a key of two parts has no module."""
    head, _, suffix = key.rpartition(".")
    module, _, leaf = head.rpartition(".")
    return module, leaf, suffix


def _key(module: str, leaf: str, suffix: str) -> str:
    return ".".join(part for part in (module, leaf, suffix) if part)


def _scope(pattern: str) -> re.Pattern:
    """A module path ending with the dotted components `pattern` matches."""
    return re.compile(rf"(?:^|\.)(?:{pattern})$")


def _leaves(weights: Mapping[str, torch.Tensor]) -> dict[tuple[str, str], dict[str, str]]:
    """(module, leaf) -> {suffix: key} over the whole dict."""
    table: dict[tuple[str, str], dict[str, str]] = defaultdict(dict)
    for key in weights:
        module, leaf, suffix = _parse(key)
        table[(module, leaf)][suffix] = key
    return table


def leaf_format(weights: Mapping[str, torch.Tensor], keys: Mapping[str, str]) -> frozenset:
    """The format of one leaf: its suffixes, each with the dtype and trailing shape of its
    tensor. Leaves of one format can share a matrix; others cannot."""
    return frozenset((suffix, weights[key].dtype, tuple(weights[key].shape[1:]))
                     for suffix, key in keys.items())


def _arrange(parts: list[torch.Tensor], how: Arrangement) -> torch.Tensor:
    if how == "rows":
        return torch.cat(parts, dim=0).contiguous()
    if how == "blocked":
        return torch.cat(parts, dim=1).contiguous()
    stacked = torch.stack(parts, dim=2)            # [experts, rows, parts, ...]
    experts, rows = stacked.shape[:2]
    return stacked.reshape(experts, rows * len(parts), *stacked.shape[3:]).contiguous()


@dataclass(frozen=True)
class Join:
    scope: str
    parts: tuple[str, ...]
    into: str
    arrange: Arrangement = "rows"

    def __call__(self, weights: Weights) -> None:
        scope = _scope(self.scope)
        table = _leaves(weights)
        owners = {module for (module, leaf) in table if leaf in self.parts and scope.search(module)}
        for module in sorted(owners):
            members = [table.get((module, part)) for part in self.parts]
            if any(not keys or "weight" not in keys for keys in members):
                continue                     # a leaf missing: nothing to fuse here
            formats = {leaf_format(weights, keys) for keys in members}
            if len(formats) > 1:             # mixed formats: one leaf each, under `into`
                for part, keys in zip(self.parts, members):
                    for suffix, key in keys.items():
                        weights[_key(f"{module}.{self.into}", part, suffix)] = weights.pop(key)
                continue
            for suffix in members[0]:
                tensors = [weights.pop(keys[suffix]) for keys in members]
                weights[_key(module, self.into, suffix)] = _arrange(tensors, self.arrange)
                del tensors


@dataclass(frozen=True)
class Stack:
    scope: str
    into: str = "switch_mlp"

    def __call__(self, weights: Weights) -> None:
        pattern = re.compile(rf"^(?P<owner>(?:.*\.)?(?:{self.scope}))\.experts\.(?P<index>\d+)$")
        groups: dict[tuple[str, str, str], dict[int, str]] = defaultdict(dict)
        for key in list(weights):
            module, leaf, suffix = _parse(key)
            found = pattern.match(module)
            if found:
                groups[(found["owner"], leaf, suffix)][int(found["index"])] = key
        for (owner, leaf, suffix), members in sorted(groups.items()):
            count = max(members) + 1
            if len(members) != count:
                raise ValueError(f"{owner}.experts: {leaf}.{suffix} is missing for experts "
                                 f"{sorted(set(range(count)) - set(members))}")
            tensors = [weights.pop(members[index]) for index in range(count)]
            weights[_key(f"{owner}.{self.into}", leaf, suffix)] = torch.stack(tensors).contiguous()
            del tensors


@dataclass(frozen=True)
class Halves:
    scope: str
    fused: str = "gate_up_proj"
    down: str = "down_proj"
    source: str = "experts"
    into: str = "switch_mlp"
    names: tuple[str, str] = ("gate_proj", "up_proj")

    def __call__(self, weights: Weights) -> None:
        scope = _scope(self.scope)
        owners = sorted({module for module, leaf, _ in map(_parse, weights)
                         if leaf == self.source and scope.search(module)})
        for owner in owners:
            fused = weights.pop(f"{owner}.{self.source}.{self.fused}", None)
            if fused is None:
                continue
            middle = fused.shape[-1] // 2
            for name, half in zip(self.names, (fused[..., :middle], fused[..., middle:])):
                weights[f"{owner}.{self.into}.{name}.weight"] = half.transpose(-2, -1).contiguous()
            del fused
            down = weights.pop(f"{owner}.{self.source}.{self.down}")
            weights[f"{owner}.{self.into}.{self.down}.weight"] = down.transpose(-2, -1).contiguous()


@dataclass(frozen=True)
class Shift:
    pattern: str
    by: float = 1.0

    def __call__(self, weights: Weights) -> None:
        pattern = re.compile(self.pattern)
        for key in [key for key in weights if pattern.search(key)]:
            weights[key] = weights[key] + self.by


@dataclass(frozen=True)
class Drop:
    pattern: str

    def __call__(self, weights: Weights) -> None:
        pattern = re.compile(self.pattern)
        for key in [key for key in weights if pattern.search(key)]:
            del weights[key]


FOLD_NORMS = Shift(r"(?:layernorm|q_norm|k_norm)\.weight$|^model\.norm\.weight$")
TIED_HEAD = Drop(r"^lm_head\.(?:weight|scales|biases)$")

LAYOUTS: dict[str, tuple[Rule, ...]] = {
    # omnia_qk_norm_rope / omnia_rope_epilogue read q, k, v as one projection.
    "qkv": (Join("self_attn", ("q_proj", "k_proj", "v_proj"), "qkv_proj"),),
    # omnia_dense_gate_up_swiglu: gate rows, then up rows, one matrix.
    "dense_gate_up": (Join("mlp", ("gate_proj", "up_proj"), "gate_up_proj"),),
    # omnia_moe_gate_up (layout="blocked"): experts stacked, each gate||up on axis 1.
    "moe_blocked": (Stack("mlp"), Join("switch_mlp", ("gate_proj", "up_proj"), "gate_up_proj", "blocked")),
    # The Core SwitchGLU order: experts stacked, gate and up rows alternating.
    "moe_interleaved": (Stack("mlp"), Join("switch_mlp", ("gate_proj", "up_proj"), "gate_up_proj",
                                           "interleaved")),
    # Experts stored pre-stacked with gate and up as halves of one [E, in, 2 * inner].
    "moe_halves": (Halves("mlp"), Join("switch_mlp", ("gate_proj", "up_proj"), "gate_up_proj", "blocked")),
    "fold_norms": (FOLD_NORMS,),
}


def apply(weights: Weights, rules: Sequence[Rule]) -> Weights:
    """Runs the rules in order over `weights` (changed in place, and returned)."""
    for rule in rules:
        rule(weights)
    return weights


def prepare(weights: Weights, rules: Sequence[Rule], *, dtype: torch.dtype | None = None,
            tie_word_embeddings: bool = False) -> Weights:
    """Casts (not a quantised checkpoint: its packed words are not numbers of a dtype),
    drops a tied head, then applies `rules`."""
    if dtype is not None:
        if any(key.endswith(".scales") for key in weights):
            raise ValueError("a quantised checkpoint (it carries .scales) cannot be cast to "
                             f"{dtype}")
        weights = {key: value.to(dtype) for key, value in weights.items()}
    if tie_word_embeddings:
        TIED_HEAD(weights)
    return apply(weights, rules)


def read_checkpoint(directory: Path | str, device: torch.device | str | None = None) -> Weights:
    """Every `model*.safetensors` shard of `directory`, merged, on `device` (the CPU when
    None)."""
    from safetensors.torch import load_file

    shards = sorted(Path(directory).glob("model*.safetensors"))
    if not shards:
        raise FileNotFoundError(f"no model*.safetensors under {directory}")
    weights: Weights = {}
    for shard in shards:
        weights.update(load_file(str(shard), device="cpu" if device is None else str(device)))
    return weights

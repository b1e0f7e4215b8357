"""The hot-path entry points as `torch.library` custom operators (`torch.ops.omnia.*`).

For callers that trace or compile (torch.compile, export): each operator is the ctypes
binding of `ops` with its outputs allocated by the operator (functional, nothing
mutated), and a fake implementation that gives the output shapes and dtypes without
touching the device. Importing this module registers them once; the facades keep
calling `ops` directly.

Registered: add_rms_norm, qk_norm_rope, rope_epilogue, embed_atlas, swiglu,
gate_softplus, gated_activations, softmax_topk, sigmoid_topk, pack_router_weight,
residual_rms_router, residual_rms_router_sigmoid; and the steps either side of the path:
moe_gate_up, moe_down_combine (dense bf16 stacks), dense_gate_up_swiglu,
dense_down_residual, attention_sink_decode.
"""

from __future__ import annotations

import torch

from . import ops

BF16 = torch.bfloat16
_LIB = "omnia"


def _op(name: str, schema_fn, fake_fn):
    op = torch.library.custom_op(f"{_LIB}::{name}", mutates_args=())(schema_fn)
    op.register_fake(fake_fn)
    return op


# add_rms_norm -------------------------------------------------------------------------

def _add_rms_norm(x: torch.Tensor, branch: torch.Tensor, weight: torch.Tensor,
                  eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    return ops.add_rms_norm(x, branch, weight, eps)


def _add_rms_norm_fake(x, branch, weight, eps):
    return torch.empty_like(x), torch.empty_like(x)


add_rms_norm = _op("add_rms_norm", _add_rms_norm, _add_rms_norm_fake)


# qk_norm_rope ---------------------------------------------------------------------------

def _qk_norm_rope(raw_queries: torch.Tensor, raw_keys: torch.Tensor, query_weight: torch.Tensor,
                  key_weight: torch.Tensor, cos_table: torch.Tensor, sin_table: torch.Tensor,
                  offset: int, eps: float, rotary_pairs: int,
                  mscale: float) -> tuple[torch.Tensor, torch.Tensor]:
    return ops.qk_norm_rope(raw_queries, raw_keys, query_weight, key_weight, cos_table, sin_table,
                            offset=offset, eps=eps, rotary_pairs=rotary_pairs, mscale=mscale)


def _qk_norm_rope_fake(raw_queries, raw_keys, query_weight, key_weight, cos_table, sin_table, offset, eps,
                       rotary_pairs, mscale):
    length, heads, dim = raw_queries.shape
    kv_heads = raw_keys.shape[1]
    return (raw_queries.new_empty((heads, length, dim), dtype=BF16),
            raw_queries.new_empty((kv_heads, length, dim), dtype=BF16))


qk_norm_rope = _op("qk_norm_rope", _qk_norm_rope, _qk_norm_rope_fake)


# rope_epilogue --------------------------------------------------------------------------

def _rope_epilogue(fused: torch.Tensor, query_weight: torch.Tensor, key_weight: torch.Tensor,
                   query_heads: int, kv_heads: int, head_dim: int, offset: int, log2_base: float,
                   eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    return ops.rope_epilogue(fused, query_weight, key_weight, query_heads=query_heads, kv_heads=kv_heads,
                             head_dim=head_dim, offset=offset, log2_base=log2_base, eps=eps)


def _rope_epilogue_fake(fused, query_weight, key_weight, query_heads, kv_heads, head_dim, offset, log2_base,
                        eps):
    length = fused.shape[0]
    return (fused.new_empty((query_heads, length, head_dim), dtype=BF16),
            fused.new_empty((kv_heads, length, head_dim), dtype=BF16))


rope_epilogue = _op("rope_epilogue", _rope_epilogue, _rope_epilogue_fake)


# embed_atlas ----------------------------------------------------------------------------

def _embed_atlas(tokens: torch.Tensor, embedding: torch.Tensor, full_atlas: torch.Tensor | None,
                 sliding_atlas: torch.Tensor | None, position: int,
                 n_positions: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Gathered rows, then the full and sliding atlas rows ([0, 0] for an atlas not given)."""
    hidden, full, sliding = ops.embed_atlas(tokens, embedding, full_atlas, sliding_atlas, position=position,
                                            n_positions=n_positions)
    # A missing atlas gets an empty tensor of its own: custom ops may not return one
    # tensor twice (the outputs would alias).
    def rows(atlas):
        return embedding.new_empty((0, 0), dtype=torch.float32) if atlas is None else atlas
    return hidden, rows(full), rows(sliding)


def _embed_atlas_fake(tokens, embedding, full_atlas, sliding_atlas, position, n_positions):
    def rows(atlas):
        if atlas is None:
            return embedding.new_empty((0, 0), dtype=torch.float32)
        return embedding.new_empty((n_positions, atlas.shape[-1]), dtype=torch.float32)
    return (embedding.new_empty((*tokens.shape, embedding.shape[1]), dtype=BF16), rows(full_atlas),
            rows(sliding_atlas))


embed_atlas = _op("embed_atlas", _embed_atlas, _embed_atlas_fake)


# activations ----------------------------------------------------------------------------

def _swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    return ops.swiglu(gate, up)


def _swiglu_fake(gate, up):
    return gate.new_empty(gate.shape, dtype=BF16)


swiglu = _op("swiglu", _swiglu, _swiglu_fake)


def _gate_softplus(a: torch.Tensor, a_log: torch.Tensor, dt_bias: torch.Tensor) -> torch.Tensor:
    return ops.gate_softplus(a, a_log, dt_bias)


def _gate_softplus_fake(a, a_log, dt_bias):
    return a.new_empty(a.shape, dtype=torch.float32)


gate_softplus = _op("gate_softplus", _gate_softplus, _gate_softplus_fake)


def _gated_activations(gate: torch.Tensor, up: torch.Tensor, a: torch.Tensor, a_log: torch.Tensor,
                       dt_bias: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    return ops.gated_activations(gate, up, a, a_log, dt_bias)


def _gated_activations_fake(gate, up, a, a_log, dt_bias):
    return gate.new_empty(gate.shape, dtype=BF16), a.new_empty(a.shape, dtype=torch.float32)


gated_activations = _op("gated_activations", _gated_activations, _gated_activations_fake)


# routing --------------------------------------------------------------------------------

def _softmax_topk(logits: torch.Tensor, k: int, normalize: bool = True,
                  shared: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    return ops.softmax_topk(logits, k, normalize=normalize, shared=shared)


def _softmax_topk_fake(logits, k, normalize=True, shared=False):
    shape = (*logits.shape[:-1], k + (1 if shared else 0))
    return logits.new_empty(shape, dtype=torch.int32), logits.new_empty(shape, dtype=torch.float32)


softmax_topk = _op("softmax_topk", _softmax_topk, _softmax_topk_fake)


def _sigmoid_topk(logits: torch.Tensor, bias: torch.Tensor, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    indices, weights, _ = ops.sigmoid_topk(logits, bias, k)
    return indices, weights


def _sigmoid_topk_fake(logits, bias, k):
    shape = (*logits.shape[:-1], k)
    return logits.new_empty(shape, dtype=torch.int32), logits.new_empty(shape, dtype=torch.float32)


sigmoid_topk = _op("sigmoid_topk", _sigmoid_topk, _sigmoid_topk_fake)


def _pack_router_weight(router_weight: torch.Tensor) -> torch.Tensor:
    return ops.pack_router_weight(router_weight).buffer


def _pack_router_weight_fake(router_weight):
    experts, hidden = router_weight.shape
    nbytes = int(ops.library().omnia_router_pack_bytes(experts, hidden))   # pure: no device
    if nbytes < 0:
        raise ValueError(f"pack_router_weight: [{experts}, {hidden}] is not served")
    return router_weight.new_empty((nbytes,), dtype=torch.uint8)


pack_router_weight = _op("pack_router_weight", _pack_router_weight, _pack_router_weight_fake)


def _residual_rms_router(x: torch.Tensor, branch: torch.Tensor, norm_weight: torch.Tensor,
                         packed: torch.Tensor, experts: int, k: int,
                         eps: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """`packed` is `pack_router_weight`'s buffer for an [experts, hidden] router."""
    router = ops.PackedRouterWeight(packed, int(experts), int(x.shape[-1]))
    summed, normalized, _, indices, weights = ops.residual_rms_router(x, branch, norm_weight, router, k=k,
                                                                      eps=eps)
    return summed, normalized, indices, weights


def _residual_rms_router_fake(x, branch, norm_weight, packed, experts, k, eps):
    shape = (*x.shape[:-1], k)
    return (torch.empty_like(x), torch.empty_like(x), x.new_empty(shape, dtype=torch.int32),
            x.new_empty(shape, dtype=torch.float32))


residual_rms_router = _op("residual_rms_router", _residual_rms_router, _residual_rms_router_fake)

def _residual_rms_router_sigmoid(x: torch.Tensor, branch: torch.Tensor, norm_weight: torch.Tensor,
                                 packed: torch.Tensor, bias: torch.Tensor, experts: int, k: int,
                                 eps: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """The reference's outputs (route/residual.py:268-299): summed, normalized, bf16 logits,
    uint32 ordinal keys; `packed` as for residual_rms_router."""
    router = ops.PackedRouterWeight(packed, int(experts), int(x.shape[-1]))
    summed, normalized, logits, keys, _, _ = ops.residual_rms_router_sigmoid(x, branch, norm_weight, router, bias,
                                                                          k=k, eps=eps)
    return summed, normalized, logits, keys


def _residual_rms_router_sigmoid_fake(x, branch, norm_weight, packed, bias, experts, k, eps):
    shape = (*x.shape[:-1], experts)
    return (torch.empty_like(x), torch.empty_like(x), x.new_empty(shape, dtype=BF16),
            x.new_empty(shape, dtype=torch.uint32))


residual_rms_router_sigmoid = _op("residual_rms_router_sigmoid", _residual_rms_router_sigmoid,
                                  _residual_rms_router_sigmoid_fake)


# the steps either side of the path ----------------------------------------------------

def _moe_gate_up(x: torch.Tensor, weight: torch.Tensor, chosen: torch.Tensor) -> torch.Tensor:
    return ops.moe_gate_up(x, weight, chosen)


def _moe_gate_up_fake(x, weight, chosen):
    return x.new_empty((chosen.numel(), weight.shape[1]), dtype=BF16)


moe_gate_up = _op("moe_gate_up", _moe_gate_up, _moe_gate_up_fake)


def _moe_down_combine(act: torch.Tensor, weight: torch.Tensor, chosen: torch.Tensor, weights: torch.Tensor,
                      residual: torch.Tensor | None) -> torch.Tensor:
    return ops.moe_down_combine(act, weight, chosen, weights, residual)


def _moe_down_combine_fake(act, weight, chosen, weights, residual):
    return act.new_empty((weight.shape[1],), dtype=BF16)


moe_down_combine = _op("moe_down_combine", _moe_down_combine, _moe_down_combine_fake)


def _dense_gate_up_swiglu(x: torch.Tensor, fused_weight: torch.Tensor) -> torch.Tensor:
    return ops.dense_gate_up_swiglu(x, fused_weight)


def _dense_gate_up_swiglu_fake(x, fused_weight):
    return x.new_empty((fused_weight.shape[0] // 2,), dtype=BF16)


dense_gate_up_swiglu = _op("dense_gate_up_swiglu", _dense_gate_up_swiglu, _dense_gate_up_swiglu_fake)


def _dense_down_residual(activated: torch.Tensor, down_weight: torch.Tensor,
                         residual: torch.Tensor) -> torch.Tensor:
    return ops.dense_down_residual(activated, down_weight, residual)


def _dense_down_residual_fake(activated, down_weight, residual):
    return activated.new_empty((down_weight.shape[0],), dtype=BF16)


dense_down_residual = _op("dense_down_residual", _dense_down_residual, _dense_down_residual_fake)


def _attention_sink_decode(queries: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, sinks: torch.Tensor,
                           mask: torch.Tensor | None, scale: float) -> torch.Tensor:
    """The cache views are read, not written; the workspace is allocated per call."""
    return ops.attention_sink_decode(queries, keys, values, sinks, mask, scale)


def _attention_sink_decode_fake(queries, keys, values, sinks, mask, scale):
    return queries.new_empty((queries.numel() // 64, 64), dtype=BF16)


attention_sink_decode = _op("attention_sink_decode", _attention_sink_decode, _attention_sink_decode_fake)

REGISTERED = ("add_rms_norm", "qk_norm_rope", "rope_epilogue", "embed_atlas", "swiglu", "gate_softplus",
              "gated_activations", "softmax_topk", "sigmoid_topk", "pack_router_weight", "residual_rms_router",
              "residual_rms_router_sigmoid", "moe_gate_up", "moe_down_combine", "dense_gate_up_swiglu",
              "dense_down_residual", "attention_sink_decode")

"""Torch-facing calls into the C ABI.

Each function checks what the kernel assumes (device, dtype, contiguity, shape),
allocates the outputs with torch on the inputs' device unless the caller passes them,
and enqueues the kernel on the current torch stream of that device. The checks run on
the host before anything is launched, so a kernel never sees a shape its grid does not
fit.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .loader import call, last_error, library

BF16 = torch.bfloat16
F32 = torch.float32


def on_rocm(*tensors: torch.Tensor) -> bool:
    """All tensors live on one ROCm device."""
    if torch.version.hip is None or not tensors:
        return False
    device = tensors[0].device
    return all(t.is_cuda and t.device == device for t in tensors)


def _require(condition: bool, message: str) -> None:
    if not condition:
        raise ValueError(message)


def _dense(t: torch.Tensor, dtype: torch.dtype, name: str) -> None:
    _require(t.dtype == dtype, f"{name}: expected {dtype}, got {t.dtype}")
    _require(t.is_contiguous(), f"{name}: must be contiguous")
    _require(t.data_ptr() % 16 == 0 or t.numel() == 0, f"{name}: must be 16-byte aligned")


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _out(out: torch.Tensor | None, like: torch.Tensor, shape, dtype, name: str) -> torch.Tensor:
    if out is None:
        return torch.empty(shape, dtype=dtype, device=like.device)
    _require(tuple(out.shape) == tuple(shape), f"{name}: shape {tuple(out.shape)} != {tuple(shape)}")
    _dense(out, dtype, name)
    _require(out.device == like.device, f"{name}: wrong device")
    return out


def rope_angle_atlas(frequencies: torch.Tensor, first: int, rows: int, *,
                     out: torch.Tensor | None = None) -> torch.Tensor:
    """Atlas rows [rows, 2 * pairs] fp32 (cos || sin) for positions first .. first+rows-1
    from fp64 frequencies [pairs] on the device; see `omnia_rope_angle_atlas`."""
    _dense(frequencies, torch.float64, "frequencies")
    pairs = frequencies.numel()
    out = _out(out, frequencies, (rows, 2 * pairs), F32, "atlas")
    _require(out.dim() == 2 and out.stride(-1) == 1 and out.shape == (rows, 2 * pairs),
             "rope_angle_atlas: out must be [rows, 2 * pairs] with unit column stride")
    _require(on_rocm(frequencies, out), "rope_angle_atlas: tensors must share one ROCm device")
    call("omnia_rope_angle_atlas", frequencies.data_ptr(), pairs, int(first), int(rows),
         out.data_ptr(), out.stride(0), _stream(frequencies))
    return out


def rope_angle_atlas_fp32(inverse_frequencies: torch.Tensor, first: int, rows: int, *,
                          out: torch.Tensor | None = None) -> torch.Tensor:
    """Atlas rows [rows, 2 * pairs] fp32 (cos || sin) in the fp32 order: theta =
    fp32(position) / inverse, from fp32 inverse frequencies [pairs] on the device; see
    `omnia_rope_angle_atlas_fp32`."""
    _dense(inverse_frequencies, F32, "inverse_frequencies")
    pairs = inverse_frequencies.numel()
    out = _out(out, inverse_frequencies, (rows, 2 * pairs), F32, "atlas")
    _require(out.dim() == 2 and out.stride(-1) == 1 and out.shape == (rows, 2 * pairs),
             "rope_angle_atlas: out must be [rows, 2 * pairs] with unit column stride")
    _require(on_rocm(inverse_frequencies, out), "rope_angle_atlas: tensors must share one ROCm device")
    call("omnia_rope_angle_atlas_fp32", inverse_frequencies.data_ptr(), pairs, int(first), int(rows),
         out.data_ptr(), out.stride(0), _stream(inverse_frequencies))
    return out


def stream_copy(src: torch.Tensor, dst: torch.Tensor, *, vectors_per_thread: int = 1) -> torch.Tensor:
    """dst <- src (same byte size, contiguous, 16-byte aligned, one ROCm device) by the
    calibration copy `omnia_stream_copy`; returns dst."""
    nbytes = src.numel() * src.element_size()
    _require(src.is_contiguous() and dst.is_contiguous(), "stream_copy: tensors must be contiguous")
    _require(dst.numel() * dst.element_size() == nbytes, "stream_copy: byte sizes differ")
    _require(on_rocm(src, dst), "stream_copy: tensors must share one ROCm device")
    call("omnia_stream_copy", src.data_ptr(), dst.data_ptr(), nbytes, int(vectors_per_thread),
         _stream(src))
    return dst


def add_rms_norm(
    x: torch.Tensor,
    branch: torch.Tensor,
    weight: torch.Tensor,
    eps: float,
    *,
    summed: torch.Tensor | None = None,
    normalized: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """`(x + branch, rms_norm(x + branch))` over the last axis; see `omnia_add_rms_norm`."""
    hidden = weight.numel()
    _require(on_rocm(x, branch, weight), "add_rms_norm: tensors must share one ROCm device")
    _require(x.shape == branch.shape and x.shape[-1] == hidden, "add_rms_norm: shape mismatch")
    for t, name in ((x, "x"), (branch, "branch"), (weight, "weight")):
        _dense(t, BF16, name)
    summed = _out(summed, x, x.shape, BF16, "summed")
    normalized = _out(normalized, x, x.shape, BF16, "normalized")
    rows = x.numel() // hidden if hidden else 0
    call(
        "omnia_add_rms_norm",
        x.data_ptr(), branch.data_ptr(), weight.data_ptr(),
        summed.data_ptr(), normalized.data_ptr(),
        rows, hidden, float(eps), _stream(x),
    )
    return summed, normalized


def _token_stride(t: torch.Tensor, name: str) -> int:
    """Token stride (elements) of a [T, H, D] view whose heads and head_dim are packed
    (a contiguous tensor, or a column slice of wider rows such as a fused qkv)."""
    _require(t.dtype == BF16, f"{name}: expected bfloat16")
    _require(t.dim() == 3, f"{name}: expected [T, H, D]")
    if t.numel() == 0:
        return t.shape[1] * t.shape[2]
    _require(t.stride(2) == 1 and t.stride(1) == t.shape[2], f"{name}: heads must be packed")
    return t.stride(0) if t.shape[0] > 1 else t.shape[1] * t.shape[2]


def qk_norm_rope(
    raw_queries: torch.Tensor,
    raw_keys: torch.Tensor,
    query_weight: torch.Tensor,
    key_weight: torch.Tensor,
    cos_table: torch.Tensor,
    sin_table: torch.Tensor,
    *,
    offset: int,
    eps: float,
    rotary_pairs: int,
    mscale: float = 1.0,
    queries: torch.Tensor | None = None,
    keys: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-head q/k RMSNorm + table RoPE; see `omnia_qk_norm_rope`.

    raw_queries [T, Hq, D] and raw_keys [T, Hkv, D] may be views with a token stride
    (e.g. slices of a fused qkv row); cos_table/sin_table are fp32 [rows, >= P] views
    with unit inner stride. Returns q [Hq, T, D] and k [Hkv, T, D].
    """
    _require(raw_queries.dim() == 3 and raw_keys.dim() == 3, "qk_norm_rope: q, k must be [T, H, D]")
    length, query_heads, head_dim = raw_queries.shape
    _require(raw_keys.shape[0] == length and raw_keys.shape[2] == head_dim, "qk_norm_rope: k shape")
    kv_heads = raw_keys.shape[1]
    _require(on_rocm(raw_queries, raw_keys, query_weight, key_weight, cos_table, sin_table),
             "qk_norm_rope: tensors must share one ROCm device")
    q_stride = _token_stride(raw_queries, "raw_queries")
    k_stride = _token_stride(raw_keys, "raw_keys")
    _dense(query_weight, BF16, "query_weight")
    _dense(key_weight, BF16, "key_weight")
    _require(query_weight.numel() == head_dim and key_weight.numel() == head_dim,
             "qk_norm_rope: norm weights must have head_dim elements")
    for table, name in ((cos_table, "cos_table"), (sin_table, "sin_table")):
        _require(table.dtype == F32 and table.dim() == 2 and table.stride(1) == 1,
                 f"{name}: fp32 [rows, width] with unit inner stride")
        _require(table.shape[1] >= rotary_pairs, f"{name}: narrower than rotary_pairs")
    _require(cos_table.shape[0] == sin_table.shape[0] and cos_table.stride(0) == sin_table.stride(0),
             "qk_norm_rope: cos and sin tables must share rows and stride")
    queries = _out(queries, raw_queries, (query_heads, length, head_dim), BF16, "queries")
    keys = _out(keys, raw_queries, (kv_heads, length, head_dim), BF16, "keys")
    call(
        "omnia_qk_norm_rope",
        raw_queries.data_ptr(), q_stride, raw_keys.data_ptr(), k_stride,
        query_weight.data_ptr(), key_weight.data_ptr(),
        cos_table.data_ptr(), sin_table.data_ptr(), cos_table.stride(0), cos_table.shape[0],
        int(offset), queries.data_ptr(), keys.data_ptr(), length,
        query_heads, kv_heads, head_dim, int(rotary_pairs), float(eps), float(mscale),
        _stream(raw_queries),
    )
    return queries, keys


def rope_epilogue(
    fused: torch.Tensor,
    query_weight: torch.Tensor,
    key_weight: torch.Tensor,
    *,
    query_heads: int,
    kv_heads: int,
    head_dim: int,
    offset: int,
    log2_base: float,
    eps: float,
    queries: torch.Tensor | None = None,
    keys: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Norm + in-kernel-angle RoPE over the q/k slices of fused qkv rows [T, W]; see
    `omnia_rope_epilogue`. Returns q [Hq, T, D] and k [Hkv, T, D]."""
    _require(fused.dim() == 2 and fused.stride(1) == 1 and fused.dtype == BF16,
             "rope_epilogue: fused must be bf16 [T, W] with unit inner stride")
    _require(on_rocm(fused, query_weight, key_weight), "rope_epilogue: tensors must share one ROCm device")
    _dense(query_weight, BF16, "query_weight")
    _dense(key_weight, BF16, "key_weight")
    length = fused.shape[0]
    queries = _out(queries, fused, (query_heads, length, head_dim), BF16, "queries")
    keys = _out(keys, fused, (kv_heads, length, head_dim), BF16, "keys")
    call(
        "omnia_rope_epilogue",
        fused.data_ptr(), fused.stride(0) if length > 1 else fused.shape[1],
        query_weight.data_ptr(), key_weight.data_ptr(), int(offset),
        queries.data_ptr(), keys.data_ptr(), length, query_heads, kv_heads, head_dim,
        float(log2_base), float(eps), _stream(fused),
    )
    return queries, keys


def embed_atlas(
    tokens: torch.Tensor,
    embedding: torch.Tensor,
    full_atlas: torch.Tensor | None,
    sliding_atlas: torch.Tensor | None,
    *,
    position: int,
    n_positions: int,
    hidden_out: torch.Tensor | None = None,
    full_out: torch.Tensor | None = None,
    sliding_out: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor | None, torch.Tensor | None]:
    """Gather `embedding[tokens]` ([*tokens.shape, H] bf16) and copy atlas rows
    position .. position+n_positions-1 ([n_positions, W] fp32); see `omnia_embed_atlas`.
    An atlas passed as None is skipped and its output is None."""
    _require(tokens.dtype == torch.int32 and tokens.is_contiguous(), "tokens: int32, contiguous")
    _require(embedding.dim() == 2, "embedding: expected [vocab, hidden]")
    _dense(embedding, BF16, "embedding")
    vocab, hidden = embedding.shape
    atlases = []
    for atlas, name in ((full_atlas, "full_atlas"), (sliding_atlas, "sliding_atlas")):
        if atlas is None:
            atlases.append((None, 0, 0))
            continue
        rows_view = atlas.reshape(-1, atlas.shape[-1])
        _dense(rows_view, F32, name)
        atlases.append((rows_view, rows_view.shape[0], rows_view.shape[1]))
    present = [t for t in (tokens, embedding, *(a for a, _, _ in atlases if a is not None))]
    _require(on_rocm(*present), "embed_atlas: tensors must share one ROCm device")
    n_tokens = tokens.numel()
    hidden_out = _out(hidden_out, embedding, (*tokens.shape, hidden), BF16, "hidden_out")
    outs = []
    for (atlas, _, width), given, name in zip(atlases, (full_out, sliding_out), ("full_out", "sliding_out")):
        outs.append(None if atlas is None else _out(given, embedding, (n_positions, width), F32, name))
    (full, full_rows, full_width), (sliding, sliding_rows, sliding_width) = atlases
    call(
        "omnia_embed_atlas",
        tokens.data_ptr(), n_tokens, embedding.data_ptr(), vocab, hidden,
        full.data_ptr() if full is not None else None, full_rows, full_width,
        sliding.data_ptr() if sliding is not None else None, sliding_rows, sliding_width,
        int(position), int(n_positions), hidden_out.data_ptr(),
        outs[0].data_ptr() if outs[0] is not None else None,
        outs[1].data_ptr() if outs[1] is not None else None,
        _stream(embedding),
    )
    return hidden_out, outs[0], outs[1]


def _row_stride(t: torch.Tensor, name: str) -> int:
    """Row stride of a [rows, width] bf16 view with unit inner stride."""
    _require(t.dim() == 2 and t.dtype == BF16, f"{name}: expected bf16 [rows, width]")
    if t.shape[0] <= 1:
        return t.shape[1]
    _require(t.stride(1) == 1, f"{name}: inner axis must be contiguous")
    return t.stride(0)


def swiglu(gate: torch.Tensor, up: torch.Tensor, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """`bf16(bf16(g * bf16(sigmoid(g))) * u)` over [..., inner]; see `omnia_swiglu`.

    gate and up may be row-strided views (e.g. the halves of a fused [T, 2I] projection)
    as long as all leading axes flatten into one row axis."""
    _require(gate.shape == up.shape, "swiglu: gate and up shapes differ")
    inner = gate.shape[-1]
    g2 = gate.reshape(-1, inner) if gate.is_contiguous() else gate
    u2 = up.reshape(-1, inner) if up.is_contiguous() else up
    if g2.dim() != 2 or u2.dim() != 2:
        g2, u2 = gate.reshape(-1, inner), up.reshape(-1, inner)
    _require(on_rocm(g2, u2), "swiglu: tensors must share one ROCm device")
    gs, us = _row_stride(g2, "gate"), _row_stride(u2, "up")
    out = _out(out, gate, gate.shape, BF16, "out")
    call("omnia_swiglu", g2.data_ptr(), gs, u2.data_ptr(), us, out.data_ptr(),
         g2.shape[0], inner, _stream(gate))
    return out


def gate_softplus(a: torch.Tensor, a_log: torch.Tensor, dt_bias: torch.Tensor, *,
                  out: torch.Tensor | None = None) -> torch.Tensor:
    """`-exp(A_log) * softplus(f32(a) + dt_bias)` over [..., heads] -> fp32; see
    `omnia_gate_softplus`."""
    heads = a.shape[-1]
    a2 = a.reshape(-1, heads) if a.is_contiguous() else a
    _require(a2.dim() == 2 and a2.dtype == BF16, "gate_softplus: a must be bf16 [rows, heads]")
    _require(a_log.shape == (heads,) and dt_bias.shape == (heads,), "gate_softplus: [heads] params")
    _dense(a_log, F32, "A_log")
    _dense(dt_bias, F32, "dt_bias")
    _require(on_rocm(a2, a_log, dt_bias), "gate_softplus: tensors must share one ROCm device")
    stride = heads if a2.shape[0] <= 1 else a2.stride(0)
    _require(a2.stride(-1) == 1, "gate_softplus: heads axis must be contiguous")
    out = _out(out, a, a.shape, F32, "out")
    call("omnia_gate_softplus", a2.data_ptr(), stride, a_log.data_ptr(), dt_bias.data_ptr(),
         out.data_ptr(), a2.shape[0], heads, _stream(a))
    return out


def gated_activations(gate: torch.Tensor, up: torch.Tensor, a: torch.Tensor,
                      a_log: torch.Tensor, dt_bias: torch.Tensor, *,
                      y: torch.Tensor | None = None,
                      g: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """`(swiglu(gate, up), gate_softplus(a, A_log, dt_bias))` in one dispatch; see
    `omnia_gated_activations`. Same operand rules as `swiglu` and `gate_softplus`, plus
    an even head count, an even row stride for `a` and 8-byte aligned A_log, dt_bias."""
    _require(gate.shape == up.shape, "gated_activations: gate and up shapes differ")
    inner = gate.shape[-1]
    g2 = gate.reshape(-1, inner) if gate.is_contiguous() else gate
    u2 = up.reshape(-1, inner) if up.is_contiguous() else up
    if g2.dim() != 2 or u2.dim() != 2:
        g2, u2 = gate.reshape(-1, inner), up.reshape(-1, inner)
    heads = a.shape[-1]
    a2 = a.reshape(-1, heads) if a.is_contiguous() else a
    _require(a2.dim() == 2 and a2.dtype == BF16, "gated_activations: a must be bf16 [rows, heads]")
    _require(a_log.shape == (heads,) and dt_bias.shape == (heads,), "gated_activations: [heads] params")
    _dense(a_log, F32, "A_log")
    _dense(dt_bias, F32, "dt_bias")
    _require(a2.stride(-1) == 1, "gated_activations: heads axis must be contiguous")
    _require(on_rocm(g2, u2, a2, a_log, dt_bias),
             "gated_activations: tensors must share one ROCm device")
    gs, us = _row_stride(g2, "gate"), _row_stride(u2, "up")
    a_stride = heads if a2.shape[0] <= 1 else a2.stride(0)
    y = _out(y, gate, gate.shape, BF16, "y")
    g = _out(g, a, a.shape, F32, "g")
    call("omnia_gated_activations", g2.data_ptr(), gs, u2.data_ptr(), us, y.data_ptr(),
         g2.shape[0], inner, a2.data_ptr(), a_stride, a_log.data_ptr(), dt_bias.data_ptr(),
         g.data_ptr(), a2.shape[0], heads, _stream(gate))
    return y, g


def gated_activations_applies(gate: torch.Tensor, up: torch.Tensor, a: torch.Tensor) -> bool:
    """The operand conditions `omnia_gated_activations` adds to swiglu's and
    gate_softplus's own: an even head count and even row stride for `a`, 4-byte alignment."""
    heads = a.shape[-1] if a.dim() else 0
    if heads == 0 or heads % 2 or a.stride(-1) != 1 or a.data_ptr() % 4:
        return False
    return a.dim() < 2 or a.shape[-2] <= 1 or a.stride(-2) % 2 == 0


def softmax_topk(logits: torch.Tensor, k: int, *, normalize: bool = True, shared: bool = False,
                 indices: torch.Tensor | None = None,
                 weights: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Top-k of bf16 router logits [..., E] (lowest index on ties) and their softmax
    weights, renormalised over the kept experts unless `normalize` is False; with
    `shared` the last logit of each row is the shared expert's gate and slot k carries
    (E - 1, its fp32 sigmoid). See `omnia_softmax_topk` / `omnia_softmax_topk_slots`.
    Returns int32 and fp32 [..., k + shared]."""
    width = logits.shape[-1]
    experts = width - (1 if shared else 0)
    rows2 = logits.reshape(-1, width) if logits.is_contiguous() else logits
    _require(rows2.dim() == 2 and rows2.dtype == BF16 and rows2.stride(-1) == 1,
             "softmax_topk: logits must be bf16 [rows, experts] with unit inner stride")
    _require(on_rocm(rows2), "softmax_topk: logits must be on a ROCm device")
    stride = width if rows2.shape[0] <= 1 else rows2.stride(0)
    shape = (*logits.shape[:-1], k + (1 if shared else 0))
    indices = _out(indices, logits, shape, torch.int32, "indices")
    weights = _out(weights, logits, shape, F32, "weights")
    if normalize and not shared:
        call("omnia_softmax_topk", rows2.data_ptr(), stride, rows2.shape[0], experts, int(k),
             indices.data_ptr(), weights.data_ptr(), _stream(logits))
    else:
        call("omnia_softmax_topk_slots", rows2.data_ptr(), stride, rows2.shape[0], experts,
             int(k), int(bool(normalize)), int(bool(shared)), indices.data_ptr(),
             weights.data_ptr(), _stream(logits))
    return indices, weights


@dataclass(frozen=True)
class PackedRouterWeight:
    """A router weight [experts, hidden] bf16 in the layout `omnia_pack_router_weight`
    writes (matrix-core operand blocks, then the fp32 row norms), on one device."""

    buffer: torch.Tensor  # uint8 [omnia_router_pack_bytes(experts, hidden)]
    experts: int
    hidden: int


def pack_router_weight(router_weight: torch.Tensor) -> PackedRouterWeight:
    """Repacks a router weight once, for `residual_rms_router`."""
    _dense(router_weight, BF16, "router_weight")
    _require(router_weight.dim() == 2, "pack_router_weight: router weight must be 2-D")
    _require(on_rocm(router_weight), "pack_router_weight: router weight must be on a ROCm device")
    experts, hidden = router_weight.shape
    nbytes = library().omnia_router_pack_bytes(experts, hidden)
    if nbytes < 0:
        raise ValueError(f"omnia_router_pack_bytes: {last_error()} (code {nbytes})")
    buffer = torch.empty(nbytes, dtype=torch.uint8, device=router_weight.device)
    call("omnia_pack_router_weight", router_weight.data_ptr(), experts, hidden,
         buffer.data_ptr(), _stream(router_weight))
    return PackedRouterWeight(buffer, int(experts), int(hidden))


# At most this many rows with the logits written out take the fused router's decode
# path: every logit an fp64 dot product spread over the chip, then the selection kernel
# (two dispatches); more rows run the fused dispatch.
ROUTER_DECODE_ROWS = 512
# A selection-only call up to this many rows is faster on the decode path (its logits
# then written to a scratch tensor) than in the fused dispatch: measured on MI355X at
# 2048 x 128, 9.9 against 13.0 us at 17 rows, 11.0 against 13.6 at 64, even at 128.
ROUTER_SELECT_VIA_DECODE_ROWS = 64


def residual_rms_router(
    x: torch.Tensor,
    branch: torch.Tensor,
    norm_weight: torch.Tensor,
    router: torch.Tensor | PackedRouterWeight,
    *,
    k: int,
    eps: float,
    emit_logits: bool = False,
    summed: torch.Tensor | None = None,
    normalized: torch.Tensor | None = None,
    logits: torch.Tensor | None = None,
    indices: torch.Tensor | None = None,
    weights: torch.Tensor | None = None,
):
    """Fused residual add + RMSNorm + router projection + top-k; see
    `omnia_residual_rms_router`. `router` is a packed weight (`pack_router_weight`, what a
    strategy holds) or the [experts, hidden] bf16 weight itself, then packed for this call.
    Returns (summed, normalized, logits or None, indices, weights). Writing the logits
    makes every logit exact: the decode path up to 512 rows, above it the fused dispatch
    with every unsure logit recomputed in fp64 (slower than selecting alone)."""
    hidden = norm_weight.numel()
    if not isinstance(router, PackedRouterWeight):
        _require(router.dim() == 2 and router.shape[-1] == hidden,
                 "residual_rms_router: router weight shape")
        router = pack_router_weight(router)
    experts = router.experts
    _require(router.hidden == hidden, "residual_rms_router: router weight shape")
    _require(x.shape == branch.shape and x.shape[-1] == hidden, "residual_rms_router: shape mismatch")
    for t, name in ((x, "x"), (branch, "branch"), (norm_weight, "norm_weight")):
        _dense(t, BF16, name)
    _require(on_rocm(x, branch, norm_weight, router.buffer),
             "residual_rms_router: tensors must share one ROCm device")
    rows = x.numel() // hidden
    lead = x.shape[:-1]
    summed = _out(summed, x, x.shape, BF16, "summed")
    normalized = _out(normalized, x, x.shape, BF16, "normalized")
    if emit_logits or logits is not None:
        logits = _out(logits, x, (*lead, experts), BF16, "logits")
    indices = _out(indices, x, (*lead, k), torch.int32, "indices")
    weights = _out(weights, x, (*lead, k), F32, "weights")
    call(
        "omnia_residual_rms_router",
        x.data_ptr(), branch.data_ptr(), norm_weight.data_ptr(), router.buffer.data_ptr(),
        rows, hidden, experts, int(k), float(eps), summed.data_ptr(), normalized.data_ptr(),
        logits.data_ptr() if logits is not None else None, indices.data_ptr(),
        weights.data_ptr(), _stream(x),
    )
    return summed, normalized, logits, indices, weights


def sigmoid_topk(logits: torch.Tensor, bias: torch.Tensor, k: int, *, emit_keys: bool = False,
                 select: bool = True, keys: torch.Tensor | None = None,
                 indices: torch.Tensor | None = None, weights: torch.Tensor | None = None):
    """Sigmoid routing with a correction bias over [..., E] bf16 or fp32 logits (rows may
    be strided); see `omnia_sigmoid_topk`. Returns (indices or None, weights or None,
    keys or None): indices int32 and weights fp32 [..., k], keys uint32 [..., E]."""
    _require(logits.dtype in (BF16, F32), "sigmoid_topk: logits must be bf16 or fp32")
    experts = logits.shape[-1]
    _require(logits.stride(-1) == 1, "sigmoid_topk: logits rows must be contiguous")
    stride = logits.stride(-2) if logits.dim() > 1 else experts
    _require(logits.dim() <= 2 or logits.is_contiguous(), "sigmoid_topk: logits must be 2-D or contiguous")
    _dense(bias, F32, "bias")
    _require(bias.numel() == experts, "sigmoid_topk: bias must be [experts]")
    _require(on_rocm(logits, bias), "sigmoid_topk: tensors must share one ROCm device")
    rows = logits.numel() // experts if logits.is_contiguous() else logits.shape[0]
    lead = logits.shape[:-1]
    if emit_keys or keys is not None:
        keys = _out(keys, logits, (*lead, experts), torch.uint32, "keys")
    if select:
        indices = _out(indices, logits, (*lead, k), torch.int32, "indices")
        weights = _out(weights, logits, (*lead, k), F32, "weights")
    else:
        indices = weights = None
    call("omnia_sigmoid_topk", logits.data_ptr(), stride, 1 if logits.dtype == F32 else 0,
         bias.data_ptr(), rows, experts, int(k), keys.data_ptr() if keys is not None else None,
         indices.data_ptr() if indices is not None else None,
         weights.data_ptr() if weights is not None else None, _stream(logits))
    return indices, weights, keys


def residual_rms_router_sigmoid(
    x: torch.Tensor,
    branch: torch.Tensor,
    norm_weight: torch.Tensor,
    router: torch.Tensor | PackedRouterWeight,
    bias: torch.Tensor,
    *,
    k: int,
    eps: float,
    emit_logits: bool = True,
    emit_keys: bool = True,
    select: bool = False,
    summed: torch.Tensor | None = None,
    normalized: torch.Tensor | None = None,
    logits: torch.Tensor | None = None,
    keys: torch.Tensor | None = None,
    indices: torch.Tensor | None = None,
    weights: torch.Tensor | None = None,
):
    """The fused router's sigmoid form; see `omnia_residual_rms_router_sigmoid`.
    Returns (summed, normalized, logits or None, keys or None, indices or None,
    weights or None); an output passed in is written in place.

    Writing the logits or the keys (the defaults: the reference's own outputs) makes
    every logit exact. Up to 512 rows that is the decode path (about 10 us at 17 rows,
    32 us at 512, at 2048 x 128); above it the fused dispatch recomputes every unsure
    logit in fp64, about 2.6 times the selection-only launch at [4096, 2048] x 128. A
    caller that only needs the selection passes emit_logits=False, emit_keys=False."""
    hidden = norm_weight.numel()
    if not isinstance(router, PackedRouterWeight):
        _require(router.dim() == 2 and router.shape[-1] == hidden,
                 "residual_rms_router_sigmoid: router weight shape")
        router = pack_router_weight(router)
    experts = router.experts
    _require(router.hidden == hidden, "residual_rms_router_sigmoid: router weight shape")
    _require(x.shape == branch.shape and x.shape[-1] == hidden,
             "residual_rms_router_sigmoid: shape mismatch")
    for t, name in ((x, "x"), (branch, "branch"), (norm_weight, "norm_weight")):
        _dense(t, BF16, name)
    _dense(bias, F32, "bias")
    _require(bias.numel() == experts, "residual_rms_router_sigmoid: bias must be [experts]")
    _require(on_rocm(x, branch, norm_weight, router.buffer, bias),
             "residual_rms_router_sigmoid: tensors must share one ROCm device")
    rows = x.numel() // hidden
    lead = x.shape[:-1]
    summed = _out(summed, x, x.shape, BF16, "summed")
    normalized = _out(normalized, x, x.shape, BF16, "normalized")
    # An output passed in is written whatever its flag says.
    logits = _out(logits, x, (*lead, experts), BF16, "logits") if emit_logits or logits is not None else None
    keys = _out(keys, x, (*lead, experts), torch.uint32, "keys") if emit_keys or keys is not None else None
    select = select or indices is not None or weights is not None
    indices = _out(indices, x, (*lead, k), torch.int32, "indices") if select else None
    weights = _out(weights, x, (*lead, k), F32, "weights") if select else None
    ptr = lambda t: t.data_ptr() if t is not None else None
    call("omnia_residual_rms_router_sigmoid", x.data_ptr(), branch.data_ptr(),
         norm_weight.data_ptr(), router.buffer.data_ptr(), bias.data_ptr(), rows, hidden,
         experts, int(k), float(eps), summed.data_ptr(), normalized.data_ptr(), ptr(logits),
         ptr(keys), ptr(indices), ptr(weights), _stream(x))
    return summed, normalized, logits, keys, indices, weights


def moe_gate_up(
    x: torch.Tensor,
    weight: torch.Tensor,
    chosen: torch.Tensor,
    *,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """One token's routed gate/up projection; see `omnia_moe_gate_up`. x [hidden] bf16,
    weight [experts, 2 * inner, hidden] bf16, chosen [k] int32 -> [k, 2 * inner] bf16."""
    _require(x.dim() == 1 or x.numel() == x.shape[-1], "moe_gate_up: x must be one row")
    _require(weight.dim() == 3 and weight.shape[-1] == x.shape[-1], "moe_gate_up: weight shape")
    _dense(x, BF16, "x")
    _dense(weight, BF16, "weight")
    _require(chosen.dtype == torch.int32 and chosen.is_contiguous() and chosen.dim() == 1,
             "moe_gate_up: chosen must be contiguous int32 [k]")
    _require(on_rocm(x, weight, chosen), "moe_gate_up: tensors must share one ROCm device")
    experts, rows, hidden = weight.shape
    k = chosen.numel()
    out = _out(out, x, (k, rows), BF16, "out")
    call("omnia_moe_gate_up", x.data_ptr(), weight.data_ptr(), experts, rows, hidden,
         chosen.data_ptr(), k, out.data_ptr(), _stream(x))
    return out


def moe_down_combine(
    act: torch.Tensor,
    weight: torch.Tensor,
    chosen: torch.Tensor,
    weights: torch.Tensor,
    residual: torch.Tensor | None = None,
    *,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """One token's routed down projection with the SwiGLU, the routing weights, the expert
    sum and the residual; see `omnia_moe_down_combine`. act [k, 2 * inner] bf16, weight
    [experts, hidden, inner] bf16, chosen [k] int32, weights [k] fp32, residual [hidden]
    bf16 or None -> [hidden] bf16."""
    _require(weight.dim() == 3, "moe_down_combine: weight must be [experts, hidden, inner]")
    experts, hidden, inner = weight.shape
    k = chosen.numel()
    _require(act.shape == (k, 2 * inner), "moe_down_combine: act must be [k, 2 * inner]")
    _dense(act, BF16, "act")
    _dense(weight, BF16, "weight")
    _require(chosen.dtype == torch.int32 and chosen.is_contiguous(), "moe_down_combine: chosen int32")
    _require(weights.dtype == F32 and weights.is_contiguous() and weights.numel() == k,
             "moe_down_combine: weights must be contiguous fp32 [k]")
    tensors = [act, weight, chosen, weights]
    if residual is not None:
        _require(residual.numel() == hidden and residual.dtype == BF16 and residual.is_contiguous(),
                 "moe_down_combine: residual must be contiguous bf16 [hidden]")
        tensors.append(residual)
    _require(on_rocm(*tensors), "moe_down_combine: tensors must share one ROCm device")
    out = _out(out, act, (hidden,), BF16, "out")
    call("omnia_moe_down_combine", act.data_ptr(), weight.data_ptr(), experts, hidden, inner,
         chosen.data_ptr(), weights.data_ptr(), k,
         residual.data_ptr() if residual is not None else None, out.data_ptr(), _stream(act))
    return out


AFFINE_BITS = (2, 3, 4, 5, 6, 8)
AFFINE_GROUPS = (32, 64, 128)


@dataclass(frozen=True)
class AffineLeaf:
    """One affine-quantized matrix set as the kernels read it: weight [..., rows,
    features * bits / 32] (int32 or uint32 words, each row a little-endian bit stream),
    scales and biases [..., rows, features / group] bf16."""

    weight: torch.Tensor
    scales: torch.Tensor
    biases: torch.Tensor
    bits: int
    group: int

    @property
    def features(self) -> int:
        return self.weight.shape[-1] * 32 // self.bits

    def check(self, rows: int, features: int, stacked: bool, name: str) -> None:
        _require(self.bits in AFFINE_BITS and self.group in AFFINE_GROUPS,
                 f"{name}: bits must be one of {AFFINE_BITS} and the group one of {AFFINE_GROUPS}")
        _require(features % self.group == 0, f"{name}: the group must divide {features}")
        dims = 3 if stacked else 2
        _require(self.weight.dim() == dims and self.scales.dim() == dims and self.biases.dim() == dims,
                 f"{name}: expected {dims}-D weight, scales and biases")
        _require(self.weight.dtype in (torch.int32, torch.uint32), f"{name}: weight must hold 32-bit words")
        _require(self.weight.is_contiguous() and self.weight.data_ptr() % 16 == 0,
                 f"{name}: weight must be contiguous and 16-byte aligned")
        lead = tuple(self.weight.shape[:-2])
        _require(tuple(self.weight.shape[-2:]) == (rows, features * self.bits // 32),
                 f"{name}: weight shape {tuple(self.weight.shape)}")
        for t, part in ((self.scales, "scales"), (self.biases, "biases")):
            _require(t.dtype == BF16 and t.is_contiguous(), f"{name}: {part} must be contiguous bf16")
            _require(tuple(t.shape) == lead + (rows, features // self.group),
                     f"{name}: {part} shape {tuple(t.shape)}")

    def tensors(self) -> list[torch.Tensor]:
        return [self.weight, self.scales, self.biases]


def _shared_args(shared: AffineLeaf | None) -> tuple:
    if shared is None:
        return (None, None, None, 0, 0)
    return (shared.weight.data_ptr(), shared.scales.data_ptr(), shared.biases.data_ptr(),
            shared.bits, shared.group)


def moe_gate_up_affine(
    x: torch.Tensor,
    leaf: AffineLeaf,
    chosen: torch.Tensor,
    *,
    limit: float | None = None,
    shared: AffineLeaf | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """One token's routed gate/up over an affine-quantized stack, the interleaved layout,
    silu fused; see `omnia_moe_gate_up_affine`. x [hidden] bf16, leaf [experts, 2 * inner,
    ...], chosen [slots] int32 (with `shared`, the last slot is the shared leaf's) ->
    [slots, inner] bf16."""
    _require(x.dim() == 1 or x.numel() == x.shape[-1], "moe_gate_up_affine: x must be one row")
    hidden = x.shape[-1]
    _dense(x, BF16, "x")
    _require(leaf.weight.dim() == 3 and leaf.weight.shape[1] % 2 == 0,
             "moe_gate_up_affine: weight must be [experts, 2 * inner, words]")
    experts, rows = leaf.weight.shape[0], leaf.weight.shape[1]
    leaf.check(rows, hidden, True, "moe_gate_up_affine")
    if shared is not None:
        shared.check(rows, hidden, False, "moe_gate_up_affine shared")
    _require(chosen.dtype == torch.int32 and chosen.is_contiguous() and chosen.dim() == 1,
             "moe_gate_up_affine: chosen must be contiguous int32 [slots]")
    _require(limit is None or limit >= 0, "moe_gate_up_affine: the limit must be non-negative")
    tensors = [x, chosen, *leaf.tensors(), *(shared.tensors() if shared is not None else [])]
    _require(on_rocm(*tensors), "moe_gate_up_affine: tensors must share one ROCm device")
    slots = chosen.numel()
    out = _out(out, x, (slots, rows // 2), BF16, "out")
    call("omnia_moe_gate_up_affine", x.data_ptr(), leaf.weight.data_ptr(), leaf.scales.data_ptr(),
         leaf.biases.data_ptr(), experts, hidden, rows // 2, leaf.bits, leaf.group,
         chosen.data_ptr(), slots, float("inf") if limit is None else float(limit),
         *_shared_args(shared), out.data_ptr(), _stream(x))
    return out


def moe_down_combine_affine(
    act: torch.Tensor,
    leaf: AffineLeaf,
    chosen: torch.Tensor,
    weights: torch.Tensor,
    residual: torch.Tensor | None = None,
    *,
    shared: AffineLeaf | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """One token's routed down projection over an affine-quantized stack, the routing
    weights, the slot sum and the residual; see `omnia_moe_down_combine_affine`. act
    [slots, inner] bf16, leaf [experts, hidden, ...], chosen [slots] int32, weights [slots]
    fp32, residual [hidden] bf16 or None -> [hidden] bf16."""
    _require(leaf.weight.dim() == 3, "moe_down_combine_affine: weight must be [experts, hidden, words]")
    experts, hidden = leaf.weight.shape[0], leaf.weight.shape[1]
    slots = chosen.numel()
    _require(act.dim() == 2 and act.shape[0] == slots, "moe_down_combine_affine: act must be [slots, inner]")
    inner = act.shape[1]
    _dense(act, BF16, "act")
    leaf.check(hidden, inner, True, "moe_down_combine_affine")
    if shared is not None:
        shared.check(hidden, inner, False, "moe_down_combine_affine shared")
    _require(chosen.dtype == torch.int32 and chosen.is_contiguous(), "moe_down_combine_affine: chosen int32")
    _require(weights.dtype == F32 and weights.is_contiguous() and weights.numel() == slots,
             "moe_down_combine_affine: weights must be contiguous fp32 [slots]")
    tensors = [act, chosen, weights, *leaf.tensors(), *(shared.tensors() if shared is not None else [])]
    if residual is not None:
        _require(residual.numel() == hidden and residual.dtype == BF16 and residual.is_contiguous(),
                 "moe_down_combine_affine: residual must be contiguous bf16 [hidden]")
        tensors.append(residual)
    _require(on_rocm(*tensors), "moe_down_combine_affine: tensors must share one ROCm device")
    out = _out(out, act, (hidden,), BF16, "out")
    call("omnia_moe_down_combine_affine", act.data_ptr(), leaf.weight.data_ptr(),
         leaf.scales.data_ptr(), leaf.biases.data_ptr(), experts, hidden, inner, leaf.bits,
         leaf.group, chosen.data_ptr(), weights.data_ptr(), slots,
         residual.data_ptr() if residual is not None else None, *_shared_args(shared),
         out.data_ptr(), _stream(act))
    return out


def dense_gate_up_swiglu(
    x: torch.Tensor,
    fused_weight: torch.Tensor,
    *,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """One token through the fused gate||up weight with the bf16 SwiGLU applied; see
    `omnia_dense_gate_up_swiglu`. x [hidden] bf16, fused_weight [2 * inner, hidden] bf16
    (gate rows first) -> [inner] bf16."""
    _require(x.dim() == 1 or x.numel() == x.shape[-1], "dense_gate_up_swiglu: x must be one row")
    _require(fused_weight.dim() == 2 and fused_weight.shape[0] % 2 == 0
             and fused_weight.shape[1] == x.shape[-1],
             "dense_gate_up_swiglu: fused_weight must be [2 * inner, hidden]")
    _dense(x, BF16, "x")
    _dense(fused_weight, BF16, "fused_weight")
    _require(on_rocm(x, fused_weight), "dense_gate_up_swiglu: tensors must share one ROCm device")
    rows, hidden = fused_weight.shape
    out = _out(out, x, (rows // 2,), BF16, "out")
    call("omnia_dense_gate_up_swiglu", x.data_ptr(), fused_weight.data_ptr(), hidden, rows // 2,
         out.data_ptr(), _stream(x))
    return out


def dense_down_residual(
    activated: torch.Tensor,
    down_weight: torch.Tensor,
    residual: torch.Tensor,
    *,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """The activation down-projected with the residual added; see
    `omnia_dense_down_residual`. activated [inner] bf16, down_weight [hidden, inner] bf16,
    residual [hidden] bf16 -> [hidden] bf16."""
    _require(down_weight.dim() == 2, "dense_down_residual: down_weight must be [hidden, inner]")
    hidden, inner = down_weight.shape
    _require(activated.numel() == inner, "dense_down_residual: activated must hold inner values")
    _require(residual.numel() == hidden, "dense_down_residual: residual must hold hidden values")
    _dense(activated, BF16, "activated")
    _dense(down_weight, BF16, "down_weight")
    _dense(residual, BF16, "residual")
    _require(on_rocm(activated, down_weight, residual),
             "dense_down_residual: tensors must share one ROCm device")
    out = _out(out, activated, (hidden,), BF16, "out")
    call("omnia_dense_down_residual", activated.data_ptr(), down_weight.data_ptr(),
         residual.data_ptr(), hidden, inner, out.data_ptr(), _stream(activated))
    return out


def attention_workspace_bytes(heads: int, kv_heads: int, head_dim: int, capacity: int) -> int:
    """Bytes of workspace `attention_decode` needs for a cache of `capacity` rows."""
    nbytes = int(library().omnia_attention_workspace_bytes(heads, kv_heads, head_dim, capacity))
    _require(nbytes >= 0, "attention_workspace_bytes: geometry not served")
    return nbytes


ATTENTION_SCRATCH_BYTES = 4 * 1024 * 1024  # OMNIA_ATTENTION_SCRATCH_BYTES


def attention_sink_workspace_bytes(heads: int, kv_heads: int, key_length: int) -> int:
    """Bytes of workspace `attention_sink_decode` needs over `key_length` keys."""
    nbytes = int(library().omnia_attention_sink_workspace_bytes(heads, kv_heads, key_length))
    _require(nbytes >= 0, "attention_sink_workspace_bytes: geometry not served")
    return nbytes


def _head_rows(t: torch.Tensor, name: str) -> tuple[int, int, int]:
    """(kv_heads, rows, head stride in elements) of a [1, kv_heads, rows, 64] or
    [kv_heads, rows, 64] bf16 view whose rows are packed (a slice of a larger buffer)."""
    _require(t.dtype == BF16, f"{name}: expected bfloat16")
    view = t[0] if t.dim() == 4 else t
    _require(view.dim() == 3 and view.shape[-1] == 64, f"{name}: expected [kv_heads, rows, 64]")
    _require(view.stride(-1) == 1 and (view.shape[1] <= 1 or view.stride(-2) == 64),
             f"{name}: rows must be packed")
    stride = view.stride(0) if view.shape[0] > 1 else view.shape[1] * 64
    _require(view.data_ptr() % 16 == 0 and stride % 8 == 0, f"{name}: must be 16-byte aligned")
    return view.shape[0], view.shape[1], stride


def attention_sink_decode(
    queries: torch.Tensor,
    keys: torch.Tensor,
    values: torch.Tensor,
    sinks: torch.Tensor,
    mask: torch.Tensor | None,
    scale: float,
    *,
    workspace: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """One query per head against the cached rows with learned sink logits; see
    `omnia_attention_sink_decode`. queries [heads, 64] (or [1, heads, 1, 64]) bf16, keys and
    values [1, kv_heads, rows, 64] bf16 views with packed rows, sinks [heads] bf16, mask
    None, a boolean band [rows] (True attends) or an additive fp32 [rows] -> [heads, 64]."""
    q = queries.reshape(-1, 64)
    heads = q.shape[0]
    _dense(q, BF16, "queries")
    kv_heads, rows, key_stride = _head_rows(keys, "keys")
    v_heads, v_rows, value_stride = _head_rows(values, "values")
    _require((v_heads, v_rows) == (kv_heads, rows), "attention_sink_decode: keys and values differ in shape")
    _require(sinks.dtype == BF16 and sinks.is_contiguous() and sinks.numel() == heads,
             "attention_sink_decode: sinks must be contiguous bf16 [heads]")
    additive = None
    if mask is not None:
        flat = mask.reshape(-1)
        _require(flat.numel() == rows, "attention_sink_decode: the mask must cover every row")
        if flat.dtype == torch.bool:
            additive = torch.where(flat, 0.0, float("-inf")).to(torch.float32)
        else:
            additive = flat.to(torch.float32).contiguous()
    nbytes = attention_sink_workspace_bytes(heads, kv_heads, rows)
    if workspace is None and nbytes:
        workspace = torch.empty(nbytes // 4, dtype=torch.float32, device=q.device)
    _require(workspace is None or workspace.numel() * workspace.element_size() >= nbytes,
             "attention_sink_decode: workspace too small")
    tensors = [q, keys, values, sinks] + ([additive] if additive is not None else []) + \
        ([workspace] if workspace is not None else [])
    _require(on_rocm(*tensors), "attention_sink_decode: tensors must share one ROCm device")
    out = _out(out, q, (heads, 64), BF16, "out")
    call("omnia_attention_sink_decode", q.data_ptr(), keys.data_ptr(), values.data_ptr(), key_stride, value_stride,
         heads, kv_heads, 64, rows, additive.data_ptr() if additive is not None else None, sinks.data_ptr(),
         float(scale), workspace.data_ptr() if workspace is not None else None,
         workspace.numel() * workspace.element_size() if workspace is not None else 0, out.data_ptr(), _stream(q))
    return out


def _attention_checks(raw_queries, raw_keys, raw_values, query_weight, key_weight, atlas,
                      key_cache, value_cache, position, heads, kv_heads, extra=()):
    head_dim = 128
    for t, name, count in ((raw_queries, "raw_queries", heads * head_dim),
                           (raw_keys, "raw_keys", kv_heads * head_dim),
                           (raw_values, "raw_values", kv_heads * head_dim)):
        _dense(t, BF16, name)
        _require(t.numel() == count, f"attention_decode: {name} must hold {count} values")
    _dense(query_weight, BF16, "query_weight")
    _dense(key_weight, BF16, "key_weight")
    _require(query_weight.numel() == head_dim and key_weight.numel() == head_dim,
             "attention_decode: norm weights must be [128]")
    _dense(atlas, F32, "atlas")
    _require(atlas.dim() == 2 and atlas.shape[1] % 2 == 0, "attention_decode: atlas must be [rows, 2P]")
    _dense(key_cache, BF16, "key_cache")
    _dense(value_cache, BF16, "value_cache")
    _require(key_cache.shape == value_cache.shape and key_cache.shape[-1] == head_dim
             and key_cache.shape[-3] == kv_heads and key_cache.numel() == kv_heads * key_cache.shape[-2] * head_dim,
             "attention_decode: caches must be [(1,) kv_heads, capacity, 128]")
    _require(position.dtype == torch.int32 and position.numel() == 1, "attention_decode: position int32 [1]")
    _require(on_rocm(raw_queries, raw_keys, raw_values, query_weight, key_weight, atlas, key_cache,
                     value_cache, position, *extra),
             "attention_decode: tensors must share one ROCm device")


def attention_decode(
    raw_queries: torch.Tensor,
    raw_keys: torch.Tensor,
    raw_values: torch.Tensor,
    query_weight: torch.Tensor,
    key_weight: torch.Tensor,
    atlas: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    position: torch.Tensor,
    *,
    heads: int,
    kv_heads: int,
    max_rows: int,
    scale: float,
    eps: float,
    mscale: float = 1.0,
    window: int = 0,
    workspace: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """One fused decode step over a KV cache; see `omnia_attention_decode`.

    raw_queries [heads * 128], raw_keys / raw_values [kv_heads * 128] bf16 (any shape with
    that many elements), weights [128] bf16, atlas [rows, 2 * pairs] fp32 (cos || sin),
    key_cache / value_cache [(1,) kv_heads, capacity, 128] bf16 (written in place),
    position: device int32 [1] (read, not advanced) -> [heads, 128] bf16."""
    head_dim = 128
    extra = ()
    if workspace is not None:
        _require(workspace.is_contiguous(), "attention_decode: workspace must be contiguous")
        extra = (workspace,)
    _attention_checks(raw_queries, raw_keys, raw_values, query_weight, key_weight, atlas,
                      key_cache, value_cache, position, heads, kv_heads, extra)
    capacity = key_cache.shape[-2]
    out = _out(out, raw_queries, (heads, head_dim), BF16, "out")
    call("omnia_attention_decode", raw_queries.data_ptr(), raw_keys.data_ptr(),
         raw_values.data_ptr(), query_weight.data_ptr(), key_weight.data_ptr(), atlas.data_ptr(),
         atlas.shape[0], atlas.shape[1] // 2, mscale, key_cache.data_ptr(),
         value_cache.data_ptr(), capacity, window, position.data_ptr(), max_rows, heads,
         kv_heads, head_dim, scale, eps,
         workspace.data_ptr() if workspace is not None else None,
         workspace.numel() * workspace.element_size() if workspace is not None else 0,
         out.data_ptr(), _stream(raw_queries))
    return out


def attention_decode_noalloc(
    raw_queries: torch.Tensor,
    raw_keys: torch.Tensor,
    raw_values: torch.Tensor,
    query_weight: torch.Tensor,
    key_weight: torch.Tensor,
    atlas: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    position: torch.Tensor,
    *,
    heads: int,
    kv_heads: int,
    max_rows: int,
    scale: float,
    eps: float,
    mscale: float = 1.0,
    window: int = 0,
    out: torch.Tensor,
) -> torch.Tensor:
    """`attention_decode` with the chunk states in the library's static device array
    (`omnia_attention_decode_noalloc`): the caller brings every buffer, `out` included, so
    the call allocates nothing. Calls that overlap on one GPU race on that array."""
    head_dim = 128
    _attention_checks(raw_queries, raw_keys, raw_values, query_weight, key_weight, atlas,
                      key_cache, value_cache, position, heads, kv_heads, (out,))
    _dense(out, BF16, "out")
    _require(out.numel() == heads * head_dim, "attention_decode_noalloc: out must hold heads * 128 values")
    capacity = key_cache.shape[-2]
    call("omnia_attention_decode_noalloc", raw_queries.data_ptr(), raw_keys.data_ptr(),
         raw_values.data_ptr(), query_weight.data_ptr(), key_weight.data_ptr(), atlas.data_ptr(),
         atlas.shape[0], atlas.shape[1] // 2, mscale, key_cache.data_ptr(),
         value_cache.data_ptr(), capacity, window, position.data_ptr(), max_rows, heads,
         kv_heads, head_dim, scale, eps, out.data_ptr(), _stream(raw_queries))
    return out


@dataclass(frozen=True)
class Mxfp4Leaf:
    """An MXFP4 matrix set as the kernels read it: weight [..., rows, features / 8]
    (int32 or uint32 words, two e2m1 codes per byte, the low nibble first), scales
    [..., rows, features / 32] uint8 (e8m0), and the projection's bias [..., rows] bf16 or
    None."""

    weight: torch.Tensor
    scales: torch.Tensor
    bias: torch.Tensor | None

    @property
    def features(self) -> int:
        return self.weight.shape[-1] * 8

    group = 32   # values per scale byte

    def check(self, rows: int, features: int, name: str) -> None:
        _require(features % 32 == 0, f"{name}: the contraction must be a multiple of 32")
        _require(self.weight.dim() == 3 and self.scales.dim() == 3, f"{name}: expected [experts, rows, ...]")
        _require(self.weight.dtype in (torch.int32, torch.uint32), f"{name}: weight must hold 32-bit words")
        _require(self.weight.is_contiguous() and self.weight.data_ptr() % 16 == 0,
                 f"{name}: weight must be contiguous and 16-byte aligned")
        experts = self.weight.shape[0]
        _require(tuple(self.weight.shape) == (experts, rows, features // 8), f"{name}: weight shape")
        _require(self.scales.dtype == torch.uint8 and self.scales.is_contiguous()
                 and tuple(self.scales.shape) == (experts, rows, features // self.group), f"{name}: scales")
        _require(self.group == 32 or self.scales.data_ptr() % 2 == 0,
                 f"{name}: the scales must be 2-byte aligned")   # read two groups at a time
        if self.bias is not None:
            _require(self.bias.dtype == BF16 and self.bias.is_contiguous()
                     and tuple(self.bias.shape) == (experts, rows), f"{name}: bias must be bf16 [experts, rows]")

    def tensors(self) -> list[torch.Tensor]:
        return [self.weight, self.scales] + ([self.bias] if self.bias is not None else [])


def moe_gate_up_mxfp4(
    x: torch.Tensor,
    leaf: Mxfp4Leaf,
    chosen: torch.Tensor,
    *,
    limit: float | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """One token's routed gate/up over an MXFP4 stack, the interleaved layout, the clamped
    swiglu_oai fused; see `omnia_moe_gate_up_mxfp4`. x [hidden] bf16, leaf [experts,
    2 * inner, ...], chosen [slots] int32 -> [slots, inner] bf16."""
    _require(x.dim() == 1 or x.numel() == x.shape[-1], "moe_gate_up_mxfp4: x must be one row")
    hidden = x.shape[-1]
    _dense(x, BF16, "x")
    _require(leaf.weight.dim() == 3 and leaf.weight.shape[1] % 2 == 0,
             "moe_gate_up_mxfp4: weight must be [experts, 2 * inner, words]")
    experts, rows = leaf.weight.shape[0], leaf.weight.shape[1]
    leaf.check(rows, hidden, "moe_gate_up_mxfp4")
    _require(chosen.dtype == torch.int32 and chosen.is_contiguous() and chosen.dim() == 1,
             "moe_gate_up_mxfp4: chosen must be contiguous int32 [slots]")
    _require(limit is None or limit >= 0, "moe_gate_up_mxfp4: the limit must be non-negative")
    _require(on_rocm(x, chosen, *leaf.tensors()), "moe_gate_up_mxfp4: tensors must share one ROCm device")
    slots = chosen.numel()
    out = _out(out, x, (slots, rows // 2), BF16, "out")
    call("omnia_moe_gate_up_mxfp4", x.data_ptr(), leaf.weight.data_ptr(), leaf.scales.data_ptr(),
         leaf.bias.data_ptr() if leaf.bias is not None else None, experts, hidden, rows // 2,
         chosen.data_ptr(), slots, float("inf") if limit is None else float(limit), out.data_ptr(),
         _stream(x))
    return out


def moe_down_combine_mxfp4(
    act: torch.Tensor,
    leaf: Mxfp4Leaf,
    chosen: torch.Tensor,
    weights: torch.Tensor,
    residual: torch.Tensor | None = None,
    *,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """One token's routed down projection over an MXFP4 stack with the projection bias, the
    routing weights, the slot sum and the residual; see `omnia_moe_down_combine_mxfp4`.
    act [slots, inner] bf16, leaf [experts, hidden, ...], chosen [slots] int32, weights
    [slots] fp32, residual [hidden] bf16 or None -> [hidden] bf16."""
    _require(leaf.weight.dim() == 3, "moe_down_combine_mxfp4: weight must be [experts, hidden, words]")
    experts, hidden = leaf.weight.shape[0], leaf.weight.shape[1]
    slots = chosen.numel()
    _require(act.dim() == 2 and act.shape[0] == slots, "moe_down_combine_mxfp4: act must be [slots, inner]")
    inner = act.shape[1]
    _dense(act, BF16, "act")
    leaf.check(hidden, inner, "moe_down_combine_mxfp4")
    _require(chosen.dtype == torch.int32 and chosen.is_contiguous(), "moe_down_combine_mxfp4: chosen int32")
    _require(weights.dtype == F32 and weights.is_contiguous() and weights.numel() == slots,
             "moe_down_combine_mxfp4: weights must be contiguous fp32 [slots]")
    tensors = [act, chosen, weights, *leaf.tensors()]
    if residual is not None:
        _require(residual.numel() == hidden and residual.dtype == BF16 and residual.is_contiguous(),
                 "moe_down_combine_mxfp4: residual must be contiguous bf16 [hidden]")
        tensors.append(residual)
    _require(on_rocm(*tensors), "moe_down_combine_mxfp4: tensors must share one ROCm device")
    out = _out(out, act, (hidden,), BF16, "out")
    call("omnia_moe_down_combine_mxfp4", act.data_ptr(), leaf.weight.data_ptr(), leaf.scales.data_ptr(),
         leaf.bias.data_ptr() if leaf.bias is not None else None, experts, hidden, inner,
         chosen.data_ptr(), weights.data_ptr(), slots,
         residual.data_ptr() if residual is not None else None, out.data_ptr(), _stream(act))
    return out


@dataclass(frozen=True)
class Nvfp4Leaf(Mxfp4Leaf):
    """An NVFP4 matrix set as the kernels read it: weight [..., rows, features / 8] (two e2m1
    codes per byte, the low nibble first), scales [..., rows, features / 16] uint8 (e4m3),
    no bias."""

    group = 16


def moe_gate_up_nvfp4(
    x: torch.Tensor,
    leaf: Nvfp4Leaf,
    chosen: torch.Tensor,
    *,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """One token's routed gate/up over an NVFP4 stack, the interleaved layout, the plain
    SwiGLU chain fused; see `omnia_moe_gate_up_nvfp4`. x [hidden] bf16, leaf [experts,
    2 * inner, ...], chosen [slots] int32 -> [slots, inner] bf16."""
    _require(x.dim() == 1 or x.numel() == x.shape[-1], "moe_gate_up_nvfp4: x must be one row")
    hidden = x.shape[-1]
    _dense(x, BF16, "x")
    _require(leaf.bias is None, "moe_gate_up_nvfp4: NVFP4 stacks carry no bias")
    _require(leaf.weight.dim() == 3 and leaf.weight.shape[1] % 2 == 0,
             "moe_gate_up_nvfp4: weight must be [experts, 2 * inner, words]")
    experts, rows = leaf.weight.shape[0], leaf.weight.shape[1]
    leaf.check(rows, hidden, "moe_gate_up_nvfp4")
    _require(chosen.dtype == torch.int32 and chosen.is_contiguous() and chosen.dim() == 1,
             "moe_gate_up_nvfp4: chosen must be contiguous int32 [slots]")
    _require(on_rocm(x, chosen, *leaf.tensors()), "moe_gate_up_nvfp4: tensors must share one ROCm device")
    slots = chosen.numel()
    out = _out(out, x, (slots, rows // 2), BF16, "out")
    call("omnia_moe_gate_up_nvfp4", x.data_ptr(), leaf.weight.data_ptr(), leaf.scales.data_ptr(), experts,
         hidden, rows // 2, chosen.data_ptr(), slots, out.data_ptr(), _stream(x))
    return out


def moe_gate_up_nvfp4_ordinal(
    x: torch.Tensor,
    leaf: Nvfp4Leaf,
    keys: torch.Tensor,
    top_k: int,
    *,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """`moe_gate_up_nvfp4` with the routing decided in the kernel: slot s runs the expert of
    rank s in the ordinal keys [experts] (ascending, equal keys to the lower index); see
    `omnia_moe_gate_up_nvfp4_ordinal`. -> [top_k, inner] bf16."""
    _require(x.dim() == 1 or x.numel() == x.shape[-1], "moe_gate_up_nvfp4_ordinal: x must be one row")
    hidden = x.shape[-1]
    _dense(x, BF16, "x")
    _require(leaf.bias is None, "moe_gate_up_nvfp4_ordinal: NVFP4 stacks carry no bias")
    _require(leaf.weight.dim() == 3 and leaf.weight.shape[1] % 2 == 0,
             "moe_gate_up_nvfp4_ordinal: weight must be [experts, 2 * inner, words]")
    experts, rows = leaf.weight.shape[0], leaf.weight.shape[1]
    leaf.check(rows, hidden, "moe_gate_up_nvfp4_ordinal")
    # The kernel ranks the keys as unsigned 32-bit values: only uint32 keys are taken, so
    # an int32 key never ranks by an order its caller did not mean.
    _require(keys.dtype == torch.uint32 and keys.is_contiguous() and keys.numel() == experts,
             "moe_gate_up_nvfp4_ordinal: keys must be contiguous uint32 [experts]")
    _require(0 < top_k <= experts <= 1024, "moe_gate_up_nvfp4_ordinal: 0 < top_k <= experts <= 1024")
    _require(on_rocm(x, keys, *leaf.tensors()), "moe_gate_up_nvfp4_ordinal: tensors must share one ROCm device")
    out = _out(out, x, (top_k, rows // 2), BF16, "out")
    call("omnia_moe_gate_up_nvfp4_ordinal", x.data_ptr(), leaf.weight.data_ptr(), leaf.scales.data_ptr(), experts,
         hidden, rows // 2, keys.data_ptr(), top_k, out.data_ptr(), _stream(x))
    return out


def moe_down_combine_nvfp4(
    act: torch.Tensor,
    leaf: Nvfp4Leaf,
    chosen: torch.Tensor,
    weights: torch.Tensor,
    residual: torch.Tensor | None = None,
    *,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """One token's routed down projection over an NVFP4 stack with the routing weights, the
    slot sum and the residual; see `omnia_moe_down_combine_nvfp4`. act [slots, inner] bf16,
    leaf [experts, hidden, ...], chosen [slots] int32, weights [slots] fp32, residual
    [hidden] bf16 or None -> [hidden] bf16."""
    _require(leaf.bias is None, "moe_down_combine_nvfp4: NVFP4 stacks carry no bias")
    _require(leaf.weight.dim() == 3, "moe_down_combine_nvfp4: weight must be [experts, hidden, words]")
    experts, hidden = leaf.weight.shape[0], leaf.weight.shape[1]
    slots = chosen.numel()
    _require(act.dim() == 2 and act.shape[0] == slots, "moe_down_combine_nvfp4: act must be [slots, inner]")
    inner = act.shape[1]
    _dense(act, BF16, "act")
    leaf.check(hidden, inner, "moe_down_combine_nvfp4")
    _require(chosen.dtype == torch.int32 and chosen.is_contiguous(), "moe_down_combine_nvfp4: chosen int32")
    _require(weights.dtype == F32 and weights.is_contiguous() and weights.numel() == slots,
             "moe_down_combine_nvfp4: weights must be contiguous fp32 [slots]")
    tensors = [act, chosen, weights, *leaf.tensors()]
    if residual is not None:
        _require(residual.numel() == hidden and residual.dtype == BF16 and residual.is_contiguous(),
                 "moe_down_combine_nvfp4: residual must be contiguous bf16 [hidden]")
        tensors.append(residual)
    _require(on_rocm(*tensors), "moe_down_combine_nvfp4: tensors must share one ROCm device")
    out = _out(out, act, (hidden,), BF16, "out")
    call("omnia_moe_down_combine_nvfp4", act.data_ptr(), leaf.weight.data_ptr(), leaf.scales.data_ptr(), experts,
         hidden, inner, chosen.data_ptr(), weights.data_ptr(), slots,
         residual.data_ptr() if residual is not None else None, out.data_ptr(), _stream(act))
    return out


def moe_down_combine_nvfp4_shared(
    act: torch.Tensor,
    leaf: Nvfp4Leaf,
    shared: Nvfp4Leaf,
    chosen: torch.Tensor,
    weights: torch.Tensor,
    residual: torch.Tensor,
    *,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """The packed NVFP4 down/combine for `tokens` tokens: the routed down projections, the
    shared stack's (the last activation row, unweighted) and the residual, with the bf16
    epilogue; see `omnia_moe_down_combine_nvfp4_shared`. act [tokens, top_k + 1, inner]
    bf16, leaf [experts, hidden, ...], shared [hidden, ...] (or [1, hidden, ...]), chosen
    [tokens, top_k] int32, weights [tokens, top_k] fp32, residual [tokens, hidden] bf16 ->
    [tokens, hidden] bf16."""
    name = "moe_down_combine_nvfp4_shared"
    _require(leaf.bias is None and shared.bias is None, f"{name}: NVFP4 stacks carry no bias")
    _require(leaf.weight.dim() == 3, f"{name}: weight must be [experts, hidden, words]")
    if shared.weight.dim() == 2:
        shared = Nvfp4Leaf(shared.weight[None], shared.scales[None], None)
    experts, hidden = leaf.weight.shape[0], leaf.weight.shape[1]
    _require(act.dim() == 3, f"{name}: act must be [tokens, top_k + 1, inner]")
    tokens, slots, inner = act.shape
    top_k = slots - 1
    _require(top_k >= 0, f"{name}: act needs the shared slot")
    _dense(act, BF16, "act")
    leaf.check(hidden, inner, name)
    shared.check(hidden, inner, name)
    _require(shared.weight.shape[0] == 1, f"{name}: the shared stack is one matrix")
    _require(chosen.dtype == torch.int32 and chosen.is_contiguous() and tuple(chosen.shape) == (tokens, top_k),
             f"{name}: chosen must be contiguous int32 [tokens, top_k]")
    _require(weights.dtype == F32 and weights.is_contiguous() and tuple(weights.shape) == (tokens, top_k),
             f"{name}: weights must be contiguous fp32 [tokens, top_k]")
    _require(residual.dtype == BF16 and residual.is_contiguous() and tuple(residual.shape) == (tokens, hidden),
             f"{name}: residual must be contiguous bf16 [tokens, hidden]")
    _require(on_rocm(act, chosen, weights, residual, *leaf.tensors(), *shared.tensors()),
             f"{name}: tensors must share one ROCm device")
    out = _out(out, act, (tokens, hidden), BF16, "out")
    call("omnia_moe_down_combine_nvfp4_shared", act.data_ptr(), leaf.weight.data_ptr(), leaf.scales.data_ptr(),
         experts, shared.weight.data_ptr(), shared.scales.data_ptr(), hidden, inner, chosen.data_ptr(),
         weights.data_ptr(), tokens, top_k, residual.data_ptr(), out.data_ptr(), _stream(act))
    return out

"""The T=1 attention step over a KV cache: raw q/k/v projections in, context out.

Mirrors core/kernels/attention/__init__.py and kernel.py (`AttentionStep`,
`AttentionStepStrategy`): the declaration carries the cache, the head geometry, the norm
gains, the rotary geometry (an angle table) and the sink logits; the first strategy
whose `build` accepts it serves the layer.

- `HipAttentionStep` (`omnia_attention_decode`, csrc/attention.hip) serves what the
  reference's `FullAttentionStep` (a fixed cache, core/kernels/attention/full.py:632-740)
  and `SlidingAttentionStep` (a ring, sliding.py:583-691) serve: bf16, head_dim 128,
  q/k norm gains, a rotary table, no sinks; one fused step that writes the new K/V row
  into the cache and reads the position on the device. A prefill (T != 1) goes to the
  Core chain, as in the reference.
- `HipSinkAttentionStep` (`omnia_attention_sink_decode`, csrc/attention_sink.hip) serves
  what the reference's `SinkAttentionStep` serves (core/kernels/attention/sink.py:256-366):
  a layer with learned sink logits over a growing `KVCache`, bf16, head_dim 64, 1, 2, 4
  or 8 query heads per kv head; the norms, the rotation and the cache write run as in the
  Core chain, then one split-K attention with the sink in the softmax's denominator. A
  prefill goes to the Core chain, as in the reference.
- `DefaultAttentionStep` is the Core chain (core/kernels/attention/default.py:85-156): the
  norms, the rotation, `cache.update_and_fetch` and attention in torch ops (fp32). It
  accepts everything, sinks included.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Protocol, runtime_checkable

import torch

from ...runtime import ops
from .._device import hip_device
from ..qkv_rope.atlas import AngleAtlas
from ..qkv_rope.kernel import AngleTable
from ..resolve import record_fallback, resolve
from .cache import FixedKVCache, KVCache, RingKVCache

__all__ = ["AttentionStep", "AttentionStepStrategy", "DefaultAttentionStep", "FixedKVCache",
           "HipAttentionStep", "HipSinkAttentionStep", "KVCache", "RingKVCache", "attention_step_applies",
           "sink_step_applies"]

HEAD_DIM = 128


@runtime_checkable
class AttentionStepStrategy(Protocol):
    def __call__(self, raw_queries: torch.Tensor, raw_keys: torch.Tensor,
                 raw_values: torch.Tensor, mask=None) -> torch.Tensor: ...


def attention_step_applies(heads: int, kv_heads: int, head_dim: int, rotary_pairs: int) -> bool:
    """head_dim 128 (a 16-lane row holds a head); grouped queries 1, 2, 4 or 8 per kv head;
    the rotated half a power-of-two number of 8-element lane slices."""
    if head_dim != HEAD_DIM or kv_heads <= 0 or heads % kv_heads != 0:
        return False
    return heads // kv_heads in (1, 2, 4, 8) and rotary_pairs in (8, 16, 32, 64)


def _split_heads(raw: torch.Tensor, count: int, head_dim: int) -> torch.Tensor:
    """[1, T, count * D] -> [1, count, T, D] (default.py:28-31)."""
    return raw.reshape(1, raw.shape[1], count, head_dim).transpose(1, 2)


def _rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """bf16(w * bf16(x * inv)), inv in fp32 (the fused kernels' rounding points)."""
    xf = x.float()
    inv = torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (weight.float() * (xf * inv).to(x.dtype).float()).to(x.dtype)


def _rotate(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, pairs: int,
            mscale: float) -> torch.Tensor:
    """Half-split rotation of the first 2P dims with the folded mscale; tail untouched."""
    factor = torch.tensor(mscale, dtype=x.dtype).float()
    a = (x[..., :pairs].float() * factor).to(x.dtype).float()
    b = (x[..., pairs : 2 * pairs].float() * factor).to(x.dtype).float()
    rotated = torch.cat([a * cos - b * sin, a * sin + b * cos], dim=-1).to(x.dtype)
    return torch.cat([rotated, x[..., 2 * pairs :]], dim=-1)


@dataclass(frozen=True)
class DefaultAttentionStep(AttentionStepStrategy):
    cache: FixedKVCache
    heads: int
    kv_heads: int
    head_dim: int
    scale: float
    query_weight: torch.Tensor | None
    key_weight: torch.Tensor | None
    eps: float
    rotary_pairs: int
    mscale: float
    angles: AngleTable | None
    base: float
    sinks: torch.Tensor | None

    @classmethod
    def build(cls, cache, *, heads, kv_heads, head_dim, scale, dtype, query_weight, key_weight,
              eps, rotary_pairs, mscale, angles, base, sinks) -> "DefaultAttentionStep":
        return cls(cache, heads, kv_heads, head_dim, scale, query_weight, key_weight, eps,
                   rotary_pairs, mscale, angles, base, sinks)

    def _angles(self, offset: int, length: int, device) -> tuple[torch.Tensor, torch.Tensor]:
        pairs = self.rotary_pairs
        if self.angles is not None:
            row = self.angles(offset, length).to(device=device, dtype=torch.float32)
            return row[:, :pairs], row[:, pairs : 2 * pairs]
        index = torch.arange(pairs, dtype=torch.float64, device=device)
        positions = torch.arange(offset, offset + length, dtype=torch.float64, device=device)
        theta = positions[:, None] * torch.exp(-torch.log(torch.tensor(self.base, dtype=torch.float64)) * index / pairs)
        return torch.cos(theta).float(), torch.sin(theta).float()

    def project(self, raw_queries, raw_keys, raw_values):
        """The step up to the attention: the normed and rotated queries [1, heads, T, D],
        and the cached keys and values once this step's rows are written."""
        position = self.cache.offset
        length = raw_queries.shape[1]
        q = _split_heads(raw_queries, self.heads, self.head_dim)
        k = _split_heads(raw_keys, self.kv_heads, self.head_dim)
        v = _split_heads(raw_values, self.kv_heads, self.head_dim)
        if self.query_weight is not None:
            q = _rms_norm(q, self.query_weight, self.eps)
        if self.key_weight is not None:
            k = _rms_norm(k, self.key_weight, self.eps)
        if self.rotary_pairs:
            cos, sin = self._angles(position, length, q.device)
            q = _rotate(q, cos, sin, self.rotary_pairs, self.mscale)
            k = _rotate(k, cos, sin, self.rotary_pairs, self.mscale)
        keys, values = self.cache.update_and_fetch(k, v)
        return q, keys, values

    def __call__(self, raw_queries, raw_keys, raw_values, mask=None):
        q, keys, values = self.project(raw_queries, raw_keys, raw_values)
        gqa = self.heads // self.kv_heads
        kf = keys.float().repeat_interleave(gqa, dim=1)
        vf = values.float().repeat_interleave(gqa, dim=1)
        scores = (q.float() @ kf.transpose(-1, -2).contiguous()) * self.scale
        if isinstance(mask, str) and mask == "causal":
            # Query i sits at row rows - T + i and sees the rows up to it.
            rows, length = scores.shape[-1], scores.shape[-2]
            seen = (torch.arange(rows, device=scores.device)[None]
                    <= (rows - length + torch.arange(length, device=scores.device))[:, None])
            scores = scores.masked_fill(~seen, float("-inf"))
        elif mask is not None and not isinstance(mask, str):
            # A boolean band attends where True (scaled_dot_product_attention's rule); a
            # float mask is additive.
            scores = (scores.masked_fill(~mask, float("-inf")) if mask.dtype == torch.bool
                      else scores + mask.float())
        if self.sinks is not None:
            sink = self.sinks.float().reshape(1, -1, 1, 1).expand(*scores.shape[:-1], 1)
            probs = torch.softmax(torch.cat([sink, scores], dim=-1), dim=-1)[..., 1:]
        else:
            probs = torch.softmax(scores, dim=-1)
        return (probs @ vf).to(raw_queries.dtype)


def capture_covered(cache: FixedKVCache, atlas_rows: int) -> None:
    """Refuse a capture whose replays could rotate at a position past the angle table.

    A replay advances the device position the host never sees. A fixed cache bounds it
    by the capacity, so the table must cover every row. A ring's position keeps rising
    past the window, so the capture needs `replay_limit` (the last position a replay
    reaches, declared with `prepare_capture`) and a table that covers it; without that
    the kernel would rotate late replays with the table's last row and no error."""
    if cache.window == 0:
        if atlas_rows < cache.capacity:
            raise ValueError(f"a captured step needs an angle table covering the cache's "
                             f"{cache.capacity} rows, not {atlas_rows}")
        return
    limit = cache.replay_limit
    if limit is None or limit < cache.offset:
        raise ValueError("a captured step over a ring cache needs the last position its "
                         "replays reach: call prepare_capture(last_position) first")
    if limit >= atlas_rows:
        raise ValueError(f"a captured step's replays reach position {limit}, past the "
                         f"angle table's {atlas_rows} rows")


@dataclass(frozen=True)
class HipAttentionStep(AttentionStepStrategy):
    cache: FixedKVCache
    heads: int
    kv_heads: int
    scale: float
    eps: float
    mscale: float
    query_weight: torch.Tensor
    key_weight: torch.Tensor
    atlas: torch.Tensor              # a fixed table's cos || sin rows
    growable: AngleAtlas | None      # or the atlas that grows past its last row
    workspace: torch.Tensor
    fallback: DefaultAttentionStep

    @classmethod
    def build(cls, cache, *, heads, kv_heads, head_dim, scale, dtype, query_weight, key_weight,
              eps, rotary_pairs, mscale, angles, base, sinks) -> "HipAttentionStep | None":
        if not isinstance(cache, FixedKVCache) or sinks is not None:
            return None
        growable = angles if isinstance(angles, AngleAtlas) else None
        if growable is not None:
            if angles.pairs != rotary_pairs:
                return None
        elif not isinstance(angles, AngleTable) or angles.pairs != rotary_pairs:
            return None
        if query_weight is None or key_weight is None:
            return None
        if dtype != torch.bfloat16 or not attention_step_applies(heads, kv_heads, head_dim, rotary_pairs):
            return None
        keys, values = cache.fetch()
        if keys.dtype != torch.bfloat16 or keys.shape[1] != kv_heads or keys.shape[3] != head_dim:
            return None
        if not (keys.is_contiguous() and values.is_contiguous()):
            return None
        if query_weight.dtype != torch.bfloat16 or key_weight.dtype != torch.bfloat16:
            return None
        table = growable.table() if growable is not None else angles
        if not hip_device(keys, values, query_weight, key_weight, table.cos, table.sin):
            return None
        atlas = (growable.atlas if growable is not None
                 else torch.cat([angles.cos, angles.sin], dim=-1).to(torch.float32).contiguous())
        nbytes = ops.attention_workspace_bytes(heads, kv_heads, head_dim, keys.shape[2])
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=keys.device)
        fallback = DefaultAttentionStep.build(
            cache, heads=heads, kv_heads=kv_heads, head_dim=head_dim, scale=scale, dtype=dtype,
            query_weight=query_weight, key_weight=key_weight, eps=eps, rotary_pairs=rotary_pairs,
            mscale=mscale, angles=angles, base=base, sinks=sinks)
        return cls(cache, heads, kv_heads, scale, eps, mscale, query_weight.contiguous(),
                   key_weight.contiguous(), atlas, growable, workspace, fallback)

    def prepare_capture(self, last_position: int) -> None:
        """Declare the last position a captured step's replays will reach, before the
        capture: a growable atlas is grown to cover it (it cannot grow inside a capture)
        and the cache records it. Replays past it are outside the contract."""
        if last_position < self.cache.offset:
            raise ValueError(f"last position {last_position} is before the cache's "
                             f"position {self.cache.offset}")
        if self.growable is not None:
            self.growable.ensure(last_position)
        self.cache.replay_limit = last_position

    def __call__(self, raw_queries, raw_keys, raw_values, mask=None):
        if raw_queries.shape[1] != 1:
            record_fallback(self, self.fallback)
            return self.fallback(raw_queries, raw_keys, raw_values, mask)
        cache = self.cache
        if cache.window == 0 and cache.offset >= cache.capacity:
            raise ValueError(f"cache of {cache.capacity} rows is full")
        # A captured step is replayed at positions the host never sees (the device position
        # advances; the host offset stays where the capture left it). The grid is then
        # sized for the whole cache and the kernel takes the attended rows from the device
        # position; a fixed cache's table must cover every row a replay can write (an
        # atlas is grown before the capture: it cannot allocate inside one).
        capturing = torch.cuda.is_current_stream_capturing()
        atlas = self.atlas
        if self.growable is not None:
            if not capturing:
                self.growable.ensure(cache.offset)  # grown past its last row, as the reference's
            atlas = self.growable.atlas
        if cache.offset >= atlas.shape[0]:
            raise ValueError(f"position {cache.offset} is past the angle table's {atlas.shape[0]} rows")
        if capturing:
            capture_covered(cache, atlas.shape[0])
        keys, values = cache.fetch()
        max_rows = cache.capacity if capturing else min(cache.offset + 1, cache.capacity)
        out = ops.attention_decode(
            raw_queries.contiguous(), raw_keys.contiguous(), raw_values.contiguous(),
            self.query_weight, self.key_weight, atlas, keys, values, cache.position,
            heads=self.heads, kv_heads=self.kv_heads, max_rows=max_rows, scale=self.scale,
            eps=self.eps, mscale=self.mscale, window=cache.window, workspace=self.workspace)
        cache.advance()
        return out.reshape(1, self.heads, 1, HEAD_DIM)


SINK_HEAD_DIM = 64


def sink_step_applies(heads: int, kv_heads: int, head_dim: int) -> bool:
    """head_dim 64; grouped queries 1, 2, 4 or 8 per kv head."""
    return (head_dim == SINK_HEAD_DIM and kv_heads > 0 and heads % kv_heads == 0
            and heads // kv_heads in (1, 2, 4, 8))


@dataclass(frozen=True)
class HipSinkAttentionStep(AttentionStepStrategy):
    """The decode step of a layer with learned sinks over a growing `KVCache`: the norms,
    the rotation and the cache write as the Core chain runs them (the reference's
    SinkAttentionStep runs them in ops too, core/kernels/attention/sink.py:330-352), then
    the attention on `omnia_attention_sink_decode`. A prefill goes to the Core chain."""

    core: DefaultAttentionStep
    sinks: torch.Tensor

    @classmethod
    def build(cls, cache, *, heads, kv_heads, head_dim, scale, dtype, query_weight, key_weight,
              eps, rotary_pairs, mscale, angles, base, sinks) -> "HipSinkAttentionStep | None":
        if not isinstance(cache, KVCache) or sinks is None or dtype != torch.bfloat16:
            return None
        if sinks.dtype != dtype or tuple(sinks.shape) != (heads,) or not hip_device(sinks):
            return None
        if not sink_step_applies(heads, kv_heads, head_dim):
            return None
        core = DefaultAttentionStep.build(
            cache, heads=heads, kv_heads=kv_heads, head_dim=head_dim, scale=scale, dtype=dtype,
            query_weight=query_weight, key_weight=key_weight, eps=eps, rotary_pairs=rotary_pairs,
            mscale=mscale, angles=angles, base=base, sinks=sinks)
        return cls(core, sinks.contiguous())

    def __call__(self, raw_queries, raw_keys, raw_values, mask=None):
        if raw_queries.shape[1] != 1:
            record_fallback(self, self.core)
            return self.core(raw_queries, raw_keys, raw_values, mask)
        q, keys, values = self.core.project(raw_queries, raw_keys, raw_values)
        if q.dtype != torch.bfloat16 or not hip_device(q, keys, values):
            raise ValueError("sink attention step: the projections must be bf16 on the sinks' device")
        band = None if isinstance(mask, str) else mask
        out = ops.attention_sink_decode(q.reshape(-1, SINK_HEAD_DIM).contiguous(), keys, values, self.sinks,
                                        band, self.core.scale)
        return out.reshape(1, self.core.heads, 1, SINK_HEAD_DIM)


_STRATEGIES = (HipAttentionStep, HipSinkAttentionStep, DefaultAttentionStep)


class AttentionStep(AttentionStepStrategy):
    """The decode step over one cache: picks its binding once, then forwards every call."""

    def __init__(self, cache, *, heads: int, kv_heads: int, head_dim: int, scale: float,
                 dtype: torch.dtype, query_weight: torch.Tensor | None = None,
                 key_weight: torch.Tensor | None = None, eps: float = 1e-6,
                 rotary_pairs: int = 0, mscale: float = 1.0, angles: AngleTable | None = None,
                 base: float = 0.0, sinks: torch.Tensor | None = None,
                 reference: bool = False) -> None:
        self.strategy: AttentionStepStrategy = resolve(
            (DefaultAttentionStep,) if reference else _STRATEGIES, cache, heads=heads,
            kv_heads=kv_heads, head_dim=head_dim, scale=scale, dtype=dtype,
            query_weight=query_weight, key_weight=key_weight, eps=eps,
            rotary_pairs=rotary_pairs, mscale=mscale, angles=angles, base=base, sinks=sinks,
        )

    def prepare_capture(self, last_position: int) -> None:
        """Before capturing a step over a ring cache: the last position its replays reach
        (the binding grows what it must to cover it)."""
        prepare = getattr(self.strategy, "prepare_capture", None)
        if prepare is not None:  # the other bindings run their replays in torch ops
            prepare(last_position)

    def __call__(self, raw_queries, raw_keys, raw_values, mask=None):
        return self.strategy(raw_queries, raw_keys, raw_values, mask)

"""HIP decode attention step (csrc/attention.hip) against the oracle (oracle/attention.py).

Mirrors the reference's tests of the fused steps (tests/test_kernel_full_fused_attention.py,
tests/test_kernel_sliding_fused_attention.py): the write rows straddling every boundary of
the kernel's tiling (a 16-lane row, a 32-row block, a 128-row chunk), partial and full
rotation, the YaRN factor; rows past the attended count never enter the result, every
row up to it does, the new K/V row lands in the cache and nothing else moves. Beyond
those: every grouped-query ratio, a long cache split over many workgroups (the combine
kernel), the ring before and after it wraps, and a captured graph replaying the step
with the position advancing on the device.

Bars: the context within the north-star bf16 bar (assert_bf16_close) with at least 99% of
elements identical to the oracle's float64 attention; the new key row within the same
bar with 99.9% identical; the value row bit-exact.
"""

import numpy as np
import pytest
import torch

from mlx_omnia_amd.kernels.attention import AttentionStep, FixedKVCache, HipAttentionStep, RingKVCache
from mlx_omnia_amd.kernels.qkv_rope import AngleTable
from mlx_omnia_amd.runtime import ops
from oracle import attention as attn
from oracle.bf16 import from_float
from oracle.rope import angle_table
from util import assert_bf16_close, bits_of, to_device

pytestmark = pytest.mark.gpu

D = 128
EPS = 1e-6
SCALE = D ** -0.5
MSCALE = 1.3465735912322998


def _atlas(rows, pairs, base=10000.0):
    cos, sin = angle_table(rows, pairs, base)
    return np.concatenate([cos, sin], axis=1).astype(np.float32)


class Case:
    def __init__(self, heads, kv_heads, capacity, pairs, seed, atlas_rows=None):
        rng = np.random.default_rng(seed)
        self.heads, self.kv_heads, self.capacity, self.pairs = heads, kv_heads, capacity, pairs
        self.raw_q = from_float(rng.standard_normal(heads * D))
        self.raw_k = from_float(rng.standard_normal(kv_heads * D))
        self.raw_v = from_float(rng.standard_normal(kv_heads * D))
        self.qw = from_float(1 + 0.1 * rng.standard_normal(D))
        self.kw = from_float(1 + 0.1 * rng.standard_normal(D))
        gen = torch.Generator(device="cuda").manual_seed(seed)
        self.kc = torch.randn((kv_heads, capacity, D), generator=gen, device="cuda").to(torch.bfloat16)
        self.vc = torch.randn((kv_heads, capacity, D), generator=gen, device="cuda").to(torch.bfloat16)
        self.atlas = _atlas(atlas_rows or max(capacity, 1024), pairs)
        self.atlas_dev = torch.from_numpy(self.atlas).cuda()
        self.workspace = torch.empty(ops.attention_workspace_bytes(heads, kv_heads, D, capacity),
                                     dtype=torch.uint8, device="cuda")

    def run(self, position, *, window=0, mscale=1.0, max_rows=None, kc=None, vc=None):
        kc = self.kc.clone() if kc is None else kc
        vc = self.vc.clone() if vc is None else vc
        if max_rows is None:
            max_rows = min(position + 1, self.capacity)
        pos = torch.tensor([position], dtype=torch.int32, device="cuda")
        out = ops.attention_decode(
            to_device(self.raw_q), to_device(self.raw_k), to_device(self.raw_v),
            to_device(self.qw), to_device(self.kw), self.atlas_dev, kc, vc, pos,
            heads=self.heads, kv_heads=self.kv_heads, max_rows=max_rows, scale=SCALE, eps=EPS,
            mscale=mscale, window=window, workspace=self.workspace)
        return bits_of(out), kc, vc

    def oracle(self, position, *, window=0, mscale=1.0, kc=None, vc=None):
        kc = bits_of(self.kc if kc is None else kc)
        vc = bits_of(self.vc if vc is None else vc)
        return attn.decode_step(self.raw_q, self.raw_k, self.raw_v, self.qw, self.kw,
                                self.atlas[position], kc, vc, position, window=window,
                                scale=SCALE, eps=EPS, pairs=self.pairs, mscale=mscale)

    def check(self, position, **kw):
        got, kc, vc = self.run(position, **kw)
        kw.pop("max_rows", None)
        want, keys, values = self.oracle(position, **kw)
        assert_bf16_close(got, want, min_exact=0.99)
        write, _ = attn.step_rows(position, self.capacity, kw.get("window", 0))
        assert_bf16_close(bits_of(kc)[:, write], keys[:, write], min_exact=0.999)
        assert np.array_equal(bits_of(vc)[:, write], values[:, write])
        others = [r for r in range(self.capacity) if r != write]
        assert np.array_equal(bits_of(kc)[:, others], bits_of(self.kc)[:, others])
        assert np.array_equal(bits_of(vc)[:, others], bits_of(self.vc)[:, others])
        return got


WRITE_IDX = (0, 1, 5, 15, 16, 31, 32, 33, 63, 64, 65, 100, 127, 128, 129, 199)


@pytest.mark.parametrize("pairs", [32, 64])
@pytest.mark.parametrize("write_idx", WRITE_IDX)
def test_fixed_cache_matches_oracle(write_idx, pairs):
    print(f"attention fixed H=8 KV=2 cap=200 pos={write_idx} P={pairs}", flush=True)
    Case(8, 2, 200, pairs, seed=write_idx).check(write_idx)


@pytest.mark.parametrize("heads,kv_heads", [(16, 16), (8, 4), (32, 8), (32, 4)])
@pytest.mark.parametrize("pairs", [8, 16, 64])
def test_grouped_query_ratios(heads, kv_heads, pairs):
    print(f"attention H={heads} KV={kv_heads} P={pairs}", flush=True)
    Case(heads, kv_heads, 300, pairs, seed=heads + kv_heads + pairs).check(257)


def test_yarn_factor_touches_the_rotated_block_only():
    print("attention mscale", flush=True)
    case = Case(8, 2, 200, 32, seed=7)
    case.check(150, mscale=MSCALE)
    _, kc, _ = case.run(150, mscale=MSCALE)
    _, plain, _ = case.run(150)
    tail = slice(64, 128)   # past 2P: the norm's output, no factor
    assert np.array_equal(bits_of(kc)[:, 150, tail], bits_of(plain)[:, 150, tail])
    assert not np.array_equal(bits_of(kc)[:, 150, :64], bits_of(plain)[:, 150, :64])


def test_rows_past_the_position_never_enter_and_every_row_up_to_it_does():
    print("attention row coverage", flush=True)
    case = Case(8, 2, 200, 64, seed=8)
    base, _, _ = case.run(120)
    poisoned_k, poisoned_v = case.kc.clone(), case.vc.clone()
    poisoned_k[:, 121:] = float("nan")
    poisoned_v[:, 121:] = float("nan")
    again, _, _ = case.run(120, kc=poisoned_k, vc=poisoned_v)
    assert np.array_equal(base, again)
    # A grid sized for the whole cache (as under graph capture) reads rows past the
    # position before it knows the position; NaN and infinite rows there still drop out.
    poisoned_k[:, 160:] = float("inf")
    poisoned_v[:, 180:] = float("-inf")
    for max_rows in (121, 160, 200):
        again, _, _ = case.run(120, kc=poisoned_k, vc=poisoned_v, max_rows=max_rows)
        assert np.array_equal(base, again), max_rows
    for row in (0, 31, 64, 119):
        moved = case.vc.clone()
        moved[:, row] += 4.0
        changed, _, _ = case.run(120, vc=moved)
        assert not np.array_equal(base, changed), row


def test_long_cache_splits_and_combines():
    print("attention long cache H=32 KV=8 cap=32768 pos=30000", flush=True)
    case = Case(32, 8, 32768, 64, seed=9, atlas_rows=32768)
    got = case.check(30000)
    # The grid sized for the whole capacity (as under graph capture) gives the same context.
    same, _, _ = case.run(30000, max_rows=32768)
    assert np.array_equal(got, same)


@pytest.mark.parametrize("position", [0, 100, 255, 256, 300, 511, 512, 1000])
def test_ring_cache(position):
    print(f"attention ring window=256 pos={position}", flush=True)
    Case(8, 2, 256, 64, seed=position + 10, atlas_rows=1024).check(position, window=256)


def test_facade_steps_through_a_fixed_cache():
    print("attention facade", flush=True)
    heads, kv_heads, capacity, pairs = 16, 4, 64, 64
    rng = np.random.default_rng(11)
    atlas = _atlas(256, pairs)
    cache = FixedKVCache.empty(kv_heads, capacity, D, device="cuda")
    ring = RingKVCache.empty(kv_heads, 32, D, device="cuda")
    qw = from_float(1 + 0.1 * rng.standard_normal(D))
    kw = from_float(1 + 0.1 * rng.standard_normal(D))
    table = AngleTable.from_atlas(torch.from_numpy(atlas).cuda())
    common = dict(heads=heads, kv_heads=kv_heads, head_dim=D, scale=SCALE, dtype=torch.bfloat16,
                  query_weight=to_device(qw), key_weight=to_device(kw), eps=EPS,
                  rotary_pairs=pairs, angles=table)
    step = AttentionStep(cache, **common)
    ring_step = AttentionStep(ring, **common)
    assert isinstance(step.strategy, HipAttentionStep)
    assert isinstance(ring_step.strategy, HipAttentionStep)
    assert not isinstance(AttentionStep(cache, **common, sinks=torch.zeros(heads, device="cuda")).strategy,
                          HipAttentionStep)
    keys = np.zeros((kv_heads, capacity, D), np.uint16)
    values = np.zeros_like(keys)
    rkeys = np.zeros((kv_heads, 32, D), np.uint16)
    rvalues = np.zeros_like(rkeys)
    for position in range(40):
        q = from_float(rng.standard_normal(heads * D))
        k = from_float(rng.standard_normal(kv_heads * D))
        v = from_float(rng.standard_normal(kv_heads * D))
        args = [to_device(x).reshape(1, 1, -1) for x in (q, k, v)]
        got = bits_of(step(*args)).reshape(heads, D)
        got_ring = bits_of(ring_step(*args)).reshape(heads, D)
        want, keys, values = attn.decode_step(q, k, v, qw, kw, atlas[position], keys, values,
                                              position, window=0, scale=SCALE, eps=EPS, pairs=pairs)
        want_ring, rkeys, rvalues = attn.decode_step(q, k, v, qw, kw, atlas[position], rkeys, rvalues,
                                                     position, window=32, scale=SCALE, eps=EPS,
                                                     pairs=pairs)
        assert_bf16_close(got, want, min_exact=0.99)
        assert_bf16_close(got_ring, want_ring, min_exact=0.99)
        keys, values = bits_of(cache.keys[0]), bits_of(cache.values[0])
        rkeys, rvalues = bits_of(ring.keys[0]), bits_of(ring.values[0])
    assert cache.offset == 40 and int(cache.position.item()) == 40
    assert ring.offset == 40 and int(ring.position.item()) == 40


def test_captured_graph_replays_with_the_device_position():
    print("attention graph replay", flush=True)
    case = Case(8, 2, 256, 64, seed=12)
    kc, vc = case.kc.clone(), case.vc.clone()
    pos = torch.tensor([10], dtype=torch.int32, device="cuda")
    inputs = [to_device(x) for x in (case.raw_q, case.raw_k, case.raw_v, case.qw, case.kw)]
    out = torch.empty((8, D), dtype=torch.bfloat16, device="cuda")
    stream = torch.cuda.Stream()

    def step():
        ops.attention_decode(*inputs, case.atlas_dev, kc, vc, pos, heads=8, kv_heads=2,
                             max_rows=256, scale=SCALE, eps=EPS, workspace=case.workspace, out=out)
        pos.add_(1)

    with torch.cuda.stream(stream):
        step()                                   # warm-up outside the capture
    torch.cuda.synchronize()
    pos.fill_(10)
    kc.copy_(case.kc)
    vc.copy_(case.vc)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step()
    torch.cuda.synchronize()
    pos.fill_(10)
    kc.copy_(case.kc)
    vc.copy_(case.vc)
    keys, values = bits_of(case.kc), bits_of(case.vc)
    for position in range(10, 14):
        graph.replay()
        torch.cuda.synchronize()
        _ = torch.ones(1000, device="cuda").sum().item()   # eager work between replays
        want, keys, values = attn.decode_step(case.raw_q, case.raw_k, case.raw_v, case.qw, case.kw,
                                              case.atlas[position], keys, values, position,
                                              window=0, scale=SCALE, eps=EPS, pairs=64)
        assert_bf16_close(bits_of(out), want, min_exact=0.99)
        assert int(pos.item()) == position + 1


@pytest.mark.parametrize("ring", [False, True])
def test_facade_step_captured_and_replayed(ring):
    """The facade's step captured once and replayed over several positions: each replay
    writes its row and attends the rows the device position gives (the grid sized for the
    whole cache under capture), with eager work between replays."""
    print(f"attention facade graph replay, ring={ring}", flush=True)
    heads, kv_heads, capacity, pairs = 8, 2, 64 if ring else 256, 64
    case = Case(heads, kv_heads, capacity, pairs, seed=13)
    start = 60 if ring else 10                      # the ring wraps during the replays
    keys = case.kc.clone().unsqueeze(0)
    values = case.vc.clone().unsqueeze(0)
    cache = (RingKVCache(keys, values, position=start) if ring
             else FixedKVCache(keys, values, position=start))
    table = AngleTable(torch.from_numpy(case.atlas[:, :pairs]).cuda(),
                       torch.from_numpy(case.atlas[:, pairs:]).cuda())
    step = AttentionStep(cache, heads=heads, kv_heads=kv_heads, head_dim=D, scale=SCALE,
                         dtype=torch.bfloat16, query_weight=to_device(case.qw),
                         key_weight=to_device(case.kw), eps=EPS, rotary_pairs=pairs, angles=table)
    assert isinstance(step.strategy, HipAttentionStep)
    q, k, v = (to_device(x).reshape(1, 1, -1) for x in (case.raw_q, case.raw_k, case.raw_v))
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        step(q, k, v)                               # warm-up outside the capture
    torch.cuda.synchronize()
    cache.offset = start
    cache.position.fill_(start)
    keys.copy_(case.kc.unsqueeze(0))
    values.copy_(case.vc.unsqueeze(0))
    if ring:
        step.prepare_capture(start + 7)             # the last position a replay reaches
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        out = step(q, k, v)
    torch.cuda.synchronize()
    cache.position.fill_(start)
    keys.copy_(case.kc.unsqueeze(0))
    values.copy_(case.vc.unsqueeze(0))
    want_keys, want_values = bits_of(case.kc), bits_of(case.vc)
    for position in range(start, start + 8):
        graph.replay()
        torch.cuda.synchronize()
        _ = torch.ones(1000, device="cuda").sum().item()   # eager work between replays
        want, want_keys, want_values = attn.decode_step(
            case.raw_q, case.raw_k, case.raw_v, case.qw, case.kw, case.atlas[position], want_keys,
            want_values, position, window=capacity if ring else 0, scale=SCALE, eps=EPS, pairs=pairs)
        assert_bf16_close(bits_of(out.reshape(heads, D)), want, min_exact=0.99)
        assert int(cache.position.item()) == position + 1
    row = (start + 7) % capacity if ring else start + 7
    assert np.array_equal(bits_of(values[0])[:, row], want_values[:, row])


def test_golden_fixture():
    from pathlib import Path

    golden = np.load(Path(__file__).parent / "golden" / "attention.npz")
    kc, vc = to_device(golden["k_cache"]), to_device(golden["v_cache"])
    out = ops.attention_decode(
        to_device(golden["raw_q"]), to_device(golden["raw_k"]), to_device(golden["raw_v"]),
        to_device(golden["q_weight"]), to_device(golden["k_weight"]),
        torch.from_numpy(golden["angles"]).cuda(), kc, vc,
        torch.from_numpy(golden["position"]).cuda(), heads=4, kv_heads=2, max_rows=40,
        scale=D ** -0.5, eps=EPS,
        workspace=torch.empty(ops.attention_workspace_bytes(4, 2, D, 40), dtype=torch.uint8, device="cuda"))
    position = int(golden["position"][0])
    assert_bf16_close(bits_of(out), golden["out"], min_exact=0.99)
    assert_bf16_close(bits_of(kc)[:, position], golden["key_row"], min_exact=0.999)
    assert np.array_equal(bits_of(vc)[:, position], golden["value_row"])

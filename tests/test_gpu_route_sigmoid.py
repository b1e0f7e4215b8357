"""Sigmoid routing with a correction bias on the GPU against the oracle.

omnia_sigmoid_topk (route/ordinal.py:200-286) and the fused router's sigmoid form
(route/residual.py:117-299), both against oracle/route.py:

- keys, indices and weights bit-exact with the oracle's correctly rounded fp32 sigmoid,
  fp32 biased sum, ordinal keys, stable selection and fp32 renormalisation, over bf16
  and fp32 logits, 32 to 1024 experts, k from 1 to 64, heavy ties and NaN rows;
- the selection without keys (on the hardware sigmoid's bounds, then the contenders'
  exact scores) bit-identical to the path that scores every expert exactly;
- the reference's tie fixture through the `Route` facade (tests/test_kernel_router_
  ordinal.py:88-142): [0, 1, 2, 3, 11, 35, 67, 99];
- the reference's separated rows with a graded bias against a float64 chain
  (test_kernel_router_ordinal.py:53-70), and the bias selecting but never weighing;
- the fused router: summed bit-exact, normalized within the bf16 bar, logits and keys
  bit-exact, the key permutation property of test_kernel_residual_rms_router.py:139-171,
  the selection bit-exact; through the `ResidualRouter` facade as well;
- the softmax kernel ranks a NaN logit last (where ordinal.py puts a NaN score).
"""

import numpy as np
import pytest
import torch

from mlx_omnia_amd.kernels.leaf import RMSNormLeaf
from mlx_omnia_amd.kernels.route import (DefaultRoute, HipOrdinalRoute, HipResidualRouter,
                                         ResidualRouter, Route, Routing)
from mlx_omnia_amd.runtime import ops
from oracle import route
from oracle.bf16 import from_float, to_f32
from util import assert_bf16_close, bits_of, to_device

pytestmark = pytest.mark.gpu

KAT_EXPECTED = [0, 1, 2, 3, 11, 35, 67, 99]


def _logits(rows, experts, seed, fp32):
    rng = np.random.default_rng(seed)
    values = (rng.standard_normal((rows, experts)) * 2.0).astype(np.float32)
    values[: min(rows, 6)] = (rng.integers(-3, 3, (min(rows, 6), experts)) * 0.5).astype(np.float32)
    if fp32:
        return values, torch.from_numpy(values).cuda()
    bits = from_float(values)
    return to_f32(bits), to_device(bits)


@pytest.mark.parametrize("experts,k", [(256, 8), (128, 16), (1024, 2), (512, 4), (64, 32),
                                       (100, 7), (32, 1), (1024, 64), (256, 64)])
@pytest.mark.parametrize("fp32", [False, True])
def test_sigmoid_topk_matches_oracle(experts, k, fp32):
    print(f"sigmoid_topk experts={experts} k={k} fp32={fp32}", flush=True)
    rows = 300
    values, logits = _logits(rows, experts, experts * 7 + k, fp32)
    rng = np.random.default_rng(experts + k)
    bias = (rng.integers(-2, 3, experts) * 0.125).astype(np.float32)
    bias[::3] = rng.standard_normal(len(bias[::3])).astype(np.float32) * 0.1
    idx, w, keys = ops.sigmoid_topk(logits, torch.from_numpy(bias).cuda(), k, emit_keys=True)
    want_idx, want_w, want_keys = route.sigmoid_topk(values, bias, k)
    assert np.array_equal(keys.cpu().numpy(), want_keys)
    assert np.array_equal(idx.cpu().numpy(), want_idx)
    assert np.array_equal(w.cpu().numpy(), want_w)


@pytest.mark.parametrize("experts,k", [(128, 8), (64, 4), (256, 16), (512, 8), (1024, 64),
                                       (128, 64), (100, 7)])
@pytest.mark.parametrize("scale,bias_scale", [(2.0, 0.1), (1e-3, 1e-3), (0.0, 0.5), (0.0, 0.0)])
def test_sigmoid_topk_selection_only_matches_keys_path(experts, k, scale, bias_scale):
    """Selection without keys ranks on the hardware sigmoid's bounds and then the
    contenders' exact scores; it must give the bits of the path that computes every
    score exactly, and the oracle's: near-tied scores (tiny logits, biases the size of
    the scores), integer ties, all-equal rows and NaN logits."""
    print(f"sigmoid_topk selection only experts={experts} k={k} scale={scale} bias={bias_scale}", flush=True)
    rows = 257
    rng = np.random.default_rng(experts * 31 + k + int(scale * 1000) + int(bias_scale * 100))
    values = (rng.standard_normal((rows, experts)) * scale).astype(np.float32)
    values[:4] = (rng.integers(-3, 3, (4, experts)) * 0.5).astype(np.float32)
    values[4, :5] = np.nan
    bits = from_float(values)
    bias = (rng.standard_normal(experts) * bias_scale).astype(np.float32)
    logits, bias_t = to_device(bits), torch.from_numpy(bias).cuda()
    idx, w, none = ops.sigmoid_topk(logits, bias_t, k)
    assert none is None
    idx_keys, w_keys, _ = ops.sigmoid_topk(logits, bias_t, k, emit_keys=True)
    want_idx, want_w, _ = route.sigmoid_topk(to_f32(bits), bias, k)
    assert np.array_equal(idx.cpu().numpy(), idx_keys.cpu().numpy())
    assert np.array_equal(w.cpu().numpy(), w_keys.cpu().numpy())
    assert np.array_equal(idx.cpu().numpy(), want_idx)
    assert np.array_equal(w.cpu().numpy(), want_w)


def test_sigmoid_topk_keys_only_strided_rows_and_nan():
    values = (np.random.default_rng(1).standard_normal((40, 300)) * 2).astype(np.float32)
    values[5, [7, 50]] = np.nan
    wide = torch.from_numpy(values).cuda()
    # 64 experts, rows 300 apart, the full order of each row: NaN last, lower index first.
    logits = wide[:, :64]
    bias = torch.zeros(64, dtype=torch.float32, device="cuda")
    idx, w, keys = ops.sigmoid_topk(logits, bias, 64, emit_keys=True)
    want_idx, want_w, want_keys = route.sigmoid_topk(values[:, :64], np.zeros(64, np.float32), 64)
    assert np.array_equal(keys.cpu().numpy(), want_keys)
    assert np.array_equal(idx.cpu().numpy(), want_idx)
    assert idx.cpu().numpy()[5, -2:].tolist() == [7, 50]
    # Keys alone over 256 experts of the same strided rows.
    bias = torch.zeros(256, dtype=torch.float32, device="cuda")
    none_idx, none_w, keys2 = ops.sigmoid_topk(wide[:, :256], bias, 8, emit_keys=True, select=False)
    _, _, want_keys2 = route.sigmoid_topk(values[:, :256], np.zeros(256, np.float32), 8)
    assert none_idx is None and none_w is None
    assert np.array_equal(keys2.cpu().numpy(), want_keys2)


@pytest.mark.parametrize("experts,k", [(256, 8), (128, 16)])
@pytest.mark.parametrize("fp32", [False, True])
def test_reference_tie_fixture_via_facade(experts, k, fp32):
    values = np.arange(experts, dtype=np.float64) * -0.5
    values[[3, 11, 35, 67, 99, 120]] = values[3]
    logits = torch.from_numpy(values.astype(np.float32)).cuda()[None]
    if not fp32:
        logits = logits.to(torch.bfloat16)
    facade = Route(None, experts=experts, k=k, scoring="sigmoid",
                   bias=torch.zeros(experts, dtype=torch.float32, device="cuda"))
    assert isinstance(facade.strategy, HipOrdinalRoute)
    idx, w = facade.rows(logits)
    assert idx.cpu().numpy()[0][:8].tolist() == KAT_EXPECTED
    assert abs(float(w.sum()) - 1.0) < 1e-6


def test_facade_binds_where_the_reference_tournament_binds():
    bias = torch.zeros(128, dtype=torch.float32, device="cuda")
    assert isinstance(Route(None, experts=128, k=8, scoring="sigmoid", bias=bias).strategy, DefaultRoute)
    assert isinstance(Route(None, experts=128, k=16, scoring="sigmoid", bias=bias).strategy, HipOrdinalRoute)
    assert isinstance(Route(None, experts=128, k=16, scoring="sigmoid", bias=bias, scale=2.0).strategy,
                      DefaultRoute)


def _f64_chain(logits_f32, bias, k):
    x = logits_f32.astype(np.float64)
    y = 1.0 / (1.0 + np.exp(np.abs(x)))
    scores = np.where(x < 0.0, y, 1.0 - y)
    chosen = np.argsort(-(scores + bias.astype(np.float64)), kind="stable", axis=-1)[:, :k]
    picked = np.take_along_axis(scores, chosen, axis=-1)
    return chosen, picked / picked.sum(axis=-1, keepdims=True)


def _graded_bias(row_f32, seed, experts=256):
    rng = np.random.default_rng(seed)
    x = row_f32.astype(np.float64)
    y = 1.0 / (1.0 + np.exp(np.abs(x)))
    scores = np.where(x < 0.0, y, 1.0 - y)
    grid = np.empty(experts)
    grid[rng.permutation(experts)] = (np.arange(experts) - experts / 2) * 4.0
    return (grid - scores).astype(np.float32)


def test_separated_rows_against_float64_chain_and_bias_never_weighs():
    for seed in range(4):
        values = (np.random.default_rng(seed).standard_normal((5, 256)) * 2.0).astype(np.float32)
        bias = _graded_bias(values[0], seed + 100)
        idx, w, _ = ops.sigmoid_topk(torch.from_numpy(values).cuda(), torch.from_numpy(bias).cuda(), 8)
        ref_idx, ref_w = _f64_chain(values, bias, 8)
        assert idx.cpu().numpy().tolist() == ref_idx.tolist()
        assert np.abs(w.cpu().numpy() - ref_w).max() < 1e-5
    base = idx.cpu().numpy()[0]
    outsider = next(e for e in range(256) if e not in set(base.tolist()))
    boosted = bias + np.where(np.arange(256) == outsider, 1e4, 0.0).astype(np.float32)
    idx, w, _ = ops.sigmoid_topk(torch.from_numpy(values).cuda(), torch.from_numpy(boosted).cuda(), 8)
    ref_idx, ref_w = _f64_chain(values, boosted, 8)
    assert idx.cpu().numpy()[0][0] == outsider and idx.cpu().numpy().tolist() == ref_idx.tolist()
    assert np.abs(w.cpu().numpy() - ref_w).max() < 1e-5


def _router_inputs(rows, hidden, experts, seed):
    rng = np.random.default_rng(seed)
    return (
        from_float(rng.standard_normal((rows, hidden), dtype=np.float32)),
        from_float(rng.standard_normal((rows, hidden), dtype=np.float32)),
        from_float(1.0 + 0.1 * rng.standard_normal(hidden)),
        from_float(0.02 * rng.standard_normal((experts, hidden), dtype=np.float32)),
        (rng.standard_normal(experts) * 0.1).astype(np.float32),
    )


@pytest.mark.parametrize("rows,hidden,experts,k", [
    (4096, 2048, 128, 8), (1, 2048, 256, 8), (37, 2048, 128, 16), (300, 4096, 128, 8),
    (20, 4096, 256, 8), (45, 2048, 128, 1), (19, 4096, 256, 64),
])
def test_residual_router_sigmoid_matches_oracle(rows, hidden, experts, k):
    print(f"residual_rms_router_sigmoid rows={rows} hidden={hidden} experts={experts} k={k}", flush=True)
    x, r, w, gate, bias = _router_inputs(rows, hidden, experts, seed=rows + hidden + experts + 1)
    s, n, logits, keys, idx, wts = ops.residual_rms_router_sigmoid(
        to_device(x), to_device(r), to_device(w), to_device(gate), torch.from_numpy(bias).cuda(),
        k=k, eps=1e-6, select=True)
    torch.cuda.synchronize()
    want = route.residual_rms_router_sigmoid(x, r, w, gate, bias, 1e-6, k)
    want_s, want_n, want_logits, want_keys, want_idx, want_w = want
    assert np.array_equal(bits_of(s), want_s)
    assert_bf16_close(bits_of(n), want_n)
    assert np.array_equal(bits_of(logits), want_logits)
    assert np.array_equal(keys.cpu().numpy(), want_keys)
    assert np.array_equal(idx.cpu().numpy(), want_idx)
    assert np.array_equal(wts.cpu().numpy(), want_w)
    # Keys alone (the reference's outputs), then the selection alone: the same bits.
    _, _, logits2, keys2, none, _ = ops.residual_rms_router_sigmoid(
        to_device(x), to_device(r), to_device(w), to_device(gate), torch.from_numpy(bias).cuda(),
        k=k, eps=1e-6)
    assert none is None and torch.equal(keys2.view(torch.int32), keys.view(torch.int32))
    assert torch.equal(logits2, logits)
    _, _, no_logits, no_keys, idx3, wts3 = ops.residual_rms_router_sigmoid(
        to_device(x), to_device(r), to_device(w), to_device(gate), torch.from_numpy(bias).cuda(),
        k=k, eps=1e-6, emit_logits=False, emit_keys=False, select=True)
    assert no_logits is None and no_keys is None
    assert torch.equal(idx3, idx) and torch.equal(wts3, wts)


@pytest.mark.parametrize("rows,hidden,experts,k,gate_scale,bias_scale", [
    (512, 2048, 128, 8, 5e-4, 0.0), (512, 2048, 256, 8, 5e-4, 1e-3), (256, 4096, 128, 16, 5e-4, 0.0),
    (512, 2048, 128, 8, 0.02, 1e-4),
])
def test_residual_router_sigmoid_selection_on_close_keys(rows, hidden, experts, k, gate_scale, bias_scale):
    """The selection alone runs on bounds of the keys and recomputes only the contenders:
    tiny logits (bf16 ties among many experts, scores within a few ulps) and biases of
    the keys' own size make most keys near the k-th, and the indices and weights must
    still be those of the exact chain."""
    print(f"sigmoid selection on close keys rows={rows} hidden={hidden} experts={experts} k={k}", flush=True)
    rng = np.random.default_rng(rows + hidden + experts + k)
    x = from_float(rng.standard_normal((rows, hidden), dtype=np.float32))
    r = from_float(rng.standard_normal((rows, hidden), dtype=np.float32))
    w = from_float(1.0 + 0.1 * rng.standard_normal(hidden))
    gate = from_float(gate_scale * rng.standard_normal((experts, hidden), dtype=np.float32))
    bias = (bias_scale * rng.standard_normal(experts)).astype(np.float32)
    _, _, _, _, idx, wts = ops.residual_rms_router_sigmoid(
        to_device(x), to_device(r), to_device(w), to_device(gate), torch.from_numpy(bias).cuda(),
        k=k, eps=1e-6, emit_logits=False, emit_keys=False, select=True)
    torch.cuda.synchronize()
    _, _, _, _, want_idx, want_w = route.residual_rms_router_sigmoid(x, r, w, gate, bias, 1e-6, k)
    assert np.array_equal(idx.cpu().numpy(), want_idx)
    assert np.array_equal(wts.cpu().numpy(), want_w)


@pytest.mark.parametrize("hidden,experts", [(2048, 256), (2048, 128)])
def test_residual_router_key_permutation_property(hidden, experts):
    x, r, w, gate, _ = _router_inputs(1, hidden, experts, seed=55)
    zero = torch.zeros(experts, dtype=torch.float32, device="cuda")
    _, _, logits, _, _, _ = ops.residual_rms_router_sigmoid(
        to_device(x), to_device(r), to_device(w), to_device(gate), zero, k=8, eps=1e-6)
    scores64 = to_f32(bits_of(logits))[0].astype(np.float64)
    scores64 = np.where(scores64 < 0, 1 / (1 + np.exp(np.abs(scores64))), 1 - 1 / (1 + np.exp(np.abs(scores64))))
    grid = np.empty(experts)
    grid[np.random.default_rng(9).permutation(experts)] = (np.arange(experts) - experts / 2) * 4.0
    bias = (grid - scores64).astype(np.float32)
    _, _, again, keys, _, _ = ops.residual_rms_router_sigmoid(
        to_device(x), to_device(r), to_device(w), to_device(gate), torch.from_numpy(bias).cuda(),
        k=8, eps=1e-6)
    assert torch.equal(again, logits)
    expected = np.argsort(-(scores64 + bias.astype(np.float64)), kind="stable")
    got = np.argsort(keys.cpu().numpy()[0].astype(np.int64), kind="stable")
    assert got.tolist() == expected.tolist()


def test_residual_router_sigmoid_facade():
    rows, hidden, experts, k = 64, 2048, 256, 8
    x, r, w, gate, bias = _router_inputs(rows, hidden, experts, seed=77)
    routing = Routing(experts=experts, k=k, scoring="sigmoid", bias=torch.from_numpy(bias).cuda())
    router = ResidualRouter(RMSNormLeaf(to_device(w), 1e-6), to_device(gate), routing=routing)
    assert isinstance(router.strategy, HipResidualRouter)
    want = route.residual_rms_router_sigmoid(x, r, w, gate, bias, 1e-6, k)
    s, n, idx, wts = router(to_device(x), to_device(r))
    assert np.array_equal(bits_of(s), want[0])
    assert np.array_equal(idx.cpu().numpy(), want[4]) and np.array_equal(wts.cpu().numpy(), want[5])
    s, n, logits, keys = router.with_keys(to_device(x), to_device(r))
    assert np.array_equal(bits_of(logits), want[2]) and np.array_equal(keys.cpu().numpy(), want[3])


def test_softmax_kernel_ranks_nan_last():
    # -0, +0, 1, NaN, -1, -inf, then 58 x -131072: the full order of the row.
    row = np.array([[0x8000, 0x0000, 0x3F80, 0x7FC0, 0xBF80, 0xFF80] + [0xC800] * 58], np.uint16)
    idx, _ = ops.softmax_topk(to_device(row), 64)
    got = idx.cpu().numpy()[0].tolist()
    assert got == route.select(row, 64)[0].tolist()
    assert got[:4] == [2, 0, 1, 4] and got[-2:] == [5, 3]

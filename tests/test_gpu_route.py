"""HIP routing kernels against the oracle.

softmax_topk: indices bit-exact (ties to the lowest index), weights within rtol 1e-5.
residual_rms_router at the config (x, residual [4096, 2048] ~N(0,1), norm weight
1 + N(0, 0.1), router [128, 2048] ~N(0, 0.02), k = 8):
  - summed bit-exact, normalized within the bf16 bar;
  - logits (when emitted) bit-exact with the oracle's correctly rounded dot products:
    the kernel refines every logit whose fp32 matrix-core value could round otherwise;
  - indices bit-exact with the full oracle chain, with and without emitted logits (only
    the decisive logits are refined then); weights within rtol 1e-5;
  - exact ties forced through the fused projection (duplicated router rows give equal
    logits whatever the accumulation order) resolve to the lowest index.
"""

import numpy as np
import pytest
import torch

from mlx_omnia_amd.kernels.leaf import RMSNormLeaf
from mlx_omnia_amd.kernels.route import HipResidualRouter, HipSoftmaxTopkRoute, ResidualRouter, Route, Routing
from mlx_omnia_amd.runtime import ops
from oracle import route
from oracle.bf16 import to_f32, from_float, ulp_distance
from util import assert_bf16_close, bits_of, to_device

pytestmark = pytest.mark.gpu

KAT_EXPECTED = [0, 1, 2, 3, 11, 35, 67, 99]


def _tied(experts):
    values = np.arange(experts, dtype=np.float64) * -0.5
    values[[3, 11, 35, 67, 99, 120]] = values[3]
    return from_float(values)[None, :]


@pytest.mark.parametrize("experts,k", [(128, 8), (256, 8), (64, 4), (100, 16), (32, 32)])
def test_softmax_topk_matches_oracle(experts, k):
    rng = np.random.default_rng(experts + k)
    logits = from_float(rng.standard_normal((1000, experts)))
    logits[:10] = from_float(rng.integers(-3, 3, (10, experts)) * 0.5)  # heavy ties
    idx, w = ops.softmax_topk(to_device(logits), k)
    want_idx, want_w = route.softmax_topk(logits, k)
    assert np.array_equal(idx.cpu().numpy(), want_idx)
    np.testing.assert_allclose(w.cpu().numpy(), want_w, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("experts", [128, 256])
def test_softmax_topk_tie_fixture_via_facade(experts):
    facade = Route(None, experts=experts, k=8)
    assert isinstance(facade.strategy, HipSoftmaxTopkRoute)
    idx, w = facade.rows(to_device(_tied(experts)))
    assert idx.cpu().numpy()[0].tolist() == KAT_EXPECTED
    assert abs(float(w.sum()) - 1.0) < 1e-6


@pytest.mark.parametrize("experts,k,normalize,shared", [
    (128, 8, True, True), (128, 8, False, False), (128, 8, False, True), (256, 8, False, True),
    (64, 4, True, True), (100, 16, False, True), (32, 32, False, False), (128, 63, True, True),
    (256, 64, False, False),
])
def test_softmax_topk_slots_matches_oracle(experts, k, normalize, shared):
    """The shared sigmoid slot and the unnormalised weights: indices bit-exact, the
    shared weight bit-exact (both correctly rounded), routed weights within rtol 1e-5."""
    print(f"softmax_topk_slots experts={experts} k={k} normalize={normalize} shared={shared}", flush=True)
    rng = np.random.default_rng(experts * 7 + k)
    logits = from_float(rng.standard_normal((777, experts + shared)) * 2)
    logits[:10] = from_float(rng.integers(-3, 3, (10, experts + shared)) * 0.5)  # heavy ties
    if shared:
        logits[10:20, experts] = from_float(np.array([0.0, -0.0, 1.5, -1.5, 30.0, -30.0, 90.0, -90.0,
                                                      1e-3, -7.25]))
    idx, w = ops.softmax_topk(to_device(logits), k, normalize=normalize, shared=shared)
    want_idx, want_w = route.softmax_topk_slots(logits, k, normalize=normalize, shared=shared)
    assert idx.shape == (777, k + shared) and idx.dtype == torch.int32
    assert np.array_equal(idx.cpu().numpy(), want_idx)
    got = w.cpu().numpy()
    np.testing.assert_allclose(got[:, :k], want_w[:, :k], rtol=1e-5, atol=1e-7)
    if shared:
        assert np.array_equal(got[:, k], want_w[:, k])


def test_softmax_topk_slots_strided_rows():
    """Rows read from a wider buffer (the row stride larger than the row's logits)."""
    rng = np.random.default_rng(91)
    wide = from_float(rng.standard_normal((300, 160)))
    view = to_device(wide)[:, :129]
    idx, w = ops.softmax_topk(view, 8, normalize=False, shared=True)
    want_idx, want_w = route.softmax_topk_slots(wide[:, :129], 8, normalize=False, shared=True)
    assert np.array_equal(idx.cpu().numpy(), want_idx)
    np.testing.assert_allclose(w.cpu().numpy(), want_w, rtol=1e-5, atol=1e-7)


def test_shared_slot_fixture_via_facade():
    """The reference's shared-slot fixture (tests/test_kernel_moe_route.py:152-177 with
    shared=True), lowest-index ties: Route(..., shared=True) binds the HIP kernel."""
    facade = Route(None, experts=128, k=8, shared=True)
    assert isinstance(facade.strategy, HipSoftmaxTopkRoute)
    logits = np.concatenate([_tied(128), from_float(np.array([[1.5]]))], axis=-1)
    idx, w = facade.rows(to_device(logits))
    assert idx.cpu().numpy()[0].tolist() == KAT_EXPECTED + [128]
    got = w.cpu().numpy()[0]
    assert got[8] == np.float32(1.0 - 1.0 / (1.0 + np.exp(1.5)))
    assert abs(float(got[:8].sum()) - 1.0) < 1e-6


def test_unnormalised_decode_step_via_facade():
    """Qwen3's decode declaration with norm_topk off: the gate on the device, one row of
    logits handed in by the caller (models/qwen3/layers/moe.py:50-64)."""
    rng = np.random.default_rng(92)
    gate = to_device(from_float(0.02 * rng.standard_normal((128, 2048))))
    x = to_device(from_float(rng.standard_normal(2048)))
    facade = Route(gate, experts=128, k=8, normalize=False)
    assert isinstance(facade.strategy, HipSoftmaxTopkRoute)
    logits = x @ gate.T
    idx, w = facade(x, logits=logits)
    want_idx, want_w = route.softmax_topk_slots(bits_of(logits)[None, :], 8, normalize=False)
    assert np.array_equal(idx.cpu().numpy(), want_idx[0])
    np.testing.assert_allclose(w.cpu().numpy(), want_w[0], rtol=1e-5, atol=1e-7)
    assert float(w.sum()) < 1.0


def _router_inputs(rows, hidden, experts, seed):
    rng = np.random.default_rng(seed)
    return (
        from_float(rng.standard_normal((rows, hidden), dtype=np.float32)),
        from_float(rng.standard_normal((rows, hidden), dtype=np.float32)),
        from_float(1.0 + 0.1 * rng.standard_normal(hidden)),
        from_float(0.02 * rng.standard_normal((experts, hidden), dtype=np.float32)),
    )


@pytest.mark.parametrize("rows,hidden,experts,k", [
    (4096, 2048, 128, 8), (1, 2048, 128, 8), (37, 2048, 128, 8), (300, 4096, 128, 8), (50, 2048, 256, 16),
    (20, 4096, 256, 8), (45, 2048, 128, 1), (64, 2048, 128, 40), (19, 4096, 256, 64), (30, 2048, 128, 64),
])
def test_residual_router_matches_oracle(rows, hidden, experts, k):
    print(f"residual_rms_router rows={rows} hidden={hidden} experts={experts} k={k}", flush=True)
    x, r, w, gate = _router_inputs(rows, hidden, experts, seed=rows + hidden + experts)
    s, n, logits, idx, wts = ops.residual_rms_router(
        to_device(x), to_device(r), to_device(w), to_device(gate), k=k, eps=1e-6, emit_logits=True)
    torch.cuda.synchronize()
    want_s, want_n, want_logits, want_idx, want_w = route.residual_rms_router(x, r, w, gate, 1e-6, k)
    assert np.array_equal(bits_of(s), want_s)
    assert_bf16_close(bits_of(n), want_n)
    # Emitted logits are the correctly rounded dot products, bit for bit.
    assert np.array_equal(bits_of(logits), want_logits)
    assert np.array_equal(idx.cpu().numpy(), want_idx)
    np.testing.assert_allclose(wts.cpu().numpy(), want_w, rtol=1e-5, atol=1e-7)
    # Without emitted logits only the decisive ones are refined: same selection.
    _, _, none, idx2, wts2 = ops.residual_rms_router(
        to_device(x), to_device(r), to_device(w), to_device(gate), k=k, eps=1e-6)
    assert none is None
    assert np.array_equal(idx2.cpu().numpy(), want_idx)
    np.testing.assert_allclose(wts2.cpu().numpy(), want_w, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("rows", [1, 2, 3, 4, 5, 9, 16, 17, 512, 513])
@pytest.mark.parametrize("hidden,experts,k", [(2048, 128, 8), (4096, 256, 8), (2048, 256, 16), (4096, 128, 64)])
def test_decode_path_equals_the_fused_dispatch(rows, hidden, experts, k):
    """Up to 512 rows with the logits written take two dispatches (the projection spread
    over the chip, then the selection kernel); without the logits the one fused dispatch
    runs (and at 513 rows both do, the one writing its logits with every unsure logit
    recomputed by its token's wave). Both forms give the same bits, and the oracle's."""
    print(f"router decode path rows={rows} hidden={hidden} experts={experts} k={k}", flush=True)
    x, r, w, gate = _router_inputs(rows, hidden, experts, seed=7 * rows + hidden + experts + k)
    xd, rd, wd = to_device(x), to_device(r), to_device(w)
    packed = ops.pack_router_weight(to_device(gate))
    s1, n1, logits, idx1, w1 = ops.residual_rms_router(xd, rd, wd, packed, k=k, eps=1e-6, emit_logits=True)
    s2, n2, none, idx2, w2 = ops.residual_rms_router(xd, rd, wd, packed, k=k, eps=1e-6)
    torch.cuda.synchronize()
    assert none is None
    for a, b in ((s1, s2), (n1, n2), (idx1, idx2), (w1, w2)):
        assert torch.equal(a, b)
    want_s, want_n, want_logits, want_idx, want_w = route.residual_rms_router(x, r, w, gate, 1e-6, k)
    assert np.array_equal(bits_of(s1), want_s)
    assert_bf16_close(bits_of(n1), want_n)
    assert np.array_equal(bits_of(logits), want_logits)
    assert np.array_equal(idx1.cpu().numpy(), want_idx)
    bias = torch.from_numpy((0.1 * np.random.default_rng(rows).standard_normal(experts)).astype(np.float32)).cuda()
    s3, n3, logits3, keys3, idx3, w3 = ops.residual_rms_router_sigmoid(xd, rd, wd, packed, bias, k=k, eps=1e-6,
                                                                       select=True)
    _, _, none, keys4, idx4, w4 = ops.residual_rms_router_sigmoid(xd, rd, wd, packed, bias, k=k, eps=1e-6,
                                                                  emit_logits=False, select=True)
    torch.cuda.synchronize()
    assert none is None
    assert torch.equal(s3, s1) and torch.equal(n3, n1) and torch.equal(logits3, logits)
    assert torch.equal(keys3.view(torch.int32), keys4.view(torch.int32))
    assert torch.equal(idx3, idx4) and torch.equal(w3, w4)
    want = route.residual_rms_router_sigmoid(x, r, w, gate, bias.cpu().numpy(), 1e-6, k)
    assert np.array_equal(keys3.cpu().numpy(), want[3])
    assert np.array_equal(idx3.cpu().numpy(), want[4])
    assert np.array_equal(w3.cpu().numpy(), want[5])


@pytest.mark.parametrize("experts,hidden", [(128, 2048), (256, 4096), (32, 96)])
def test_pack_router_weight_layout_and_norms(experts, hidden):
    rng = np.random.default_rng(experts + hidden)
    gate = from_float(0.02 * rng.standard_normal((experts, hidden), dtype=np.float32))
    gate[0, :5] = from_float(np.array([0.0, -0.0, 1e-38, 3e38, -2.5], dtype=np.float32))
    packed = ops.pack_router_weight(to_device(gate))
    torch.cuda.synchronize()
    raw = packed.buffer.cpu().numpy()
    body = raw[: experts * hidden * 2].view(np.uint16).reshape(experts // 16, hidden // 32, 64, 8)
    lane = np.arange(64)
    for tile in range(experts // 16):
        for step in range(hidden // 32):
            rows = tile * 16 + lane % 16
            cols = step * 32 + (lane // 16)[:, None] * 8 + np.arange(8)[None, :]
            assert np.array_equal(body[tile, step], gate[rows[:, None], cols])
    norms = raw[experts * hidden * 2 : experts * hidden * 2 + experts * 4].view(np.float32)
    rows = raw[experts * hidden * 2 + experts * 4 :].view(np.uint16).reshape(experts, hidden)
    assert np.array_equal(rows, gate)
    exact = np.sqrt((to_f32(gate).astype(np.float64) ** 2).sum(axis=1))
    assert np.all(norms.astype(np.float64) >= exact)
    assert np.allclose(norms, exact, rtol=1e-6)


def test_residual_router_forced_ties_and_facade():
    rows, hidden, experts = 64, 2048, 128
    x, r, w, gate = _router_inputs(rows, hidden, experts, seed=9)
    # Equal router rows give equal logits: experts 3, 11, 35, 67, 99, 120 tie with 3.
    # Positive inputs and a positive offset on those rows put the group on top.
    rng = np.random.default_rng(10)
    x = from_float(np.abs(rng.standard_normal((rows, hidden))) + 1.0)
    r = from_float(0.01 * rng.standard_normal((rows, hidden)))
    base = 0.02 * rng.standard_normal(hidden)
    gate = from_float(np.tile(0.02 * rng.standard_normal(hidden), (experts, 1)) * 0.1)
    gate[[3, 11, 35, 67, 99, 120]] = from_float(base + 0.05)
    router = ResidualRouter(RMSNormLeaf(to_device(w), 1e-6), to_device(gate), routing=Routing(experts=experts, k=4))
    assert isinstance(router.strategy, HipResidualRouter)
    _, _, idx, _ = router(to_device(x), to_device(r))
    got = idx.cpu().numpy()
    assert (got == np.array([3, 11, 35, 67])).all(axis=-1).all()


def test_golden_fixture():
    golden = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "route.npz")
    idx, w = ops.softmax_topk(to_device(golden["logits"]), int(golden["k"]))
    assert np.array_equal(idx.cpu().numpy(), golden["indices"])
    np.testing.assert_allclose(w.cpu().numpy(), golden["weights"], rtol=1e-5, atol=1e-7)

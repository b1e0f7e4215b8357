"""Pins the routing oracle (oracle/route.py) independently of its formula.

- the reference's tie fixtures (tests/test_kernel_moe_route.py:152-177 for 128 experts,
  tests/test_kernel_router_ordinal.py:88-142 for 256): strictly decreasing logits with
  indices 3, 11, 35, 67, 99, 120 forced equal, so the k=8 cut falls inside the tie
  group; with the lowest-index rule the answer is [0, 1, 2, 3, 11, 35, 67, 99] (the
  reference's softmax chain, which breaks ties upward, gives [0, 1, 2, 120, 99, 67, 35,
  11] — also checked, against a brute force of that rule);
- selection against a brute-force Python sort and against torch's stable sort;
- weights: descending, summing to one, equal to torch's float64 softmax renormalised;
- logits against torch's bf16 matmul (a different accumulation), within one bf16 ulp;
- -0 and +0 tie; a NaN logit ranks last (where route/ordinal.py:37-47 puts a NaN
  score);
- planted mistakes (upward ties, no renormalisation, ascending order) fail.

The shared slot and `normalize=False` (`softmax_topk_slots`):

- the reference's shared-slot fixture (tests/test_kernel_moe_route.py:152-177 with
  shared=True: the tie fixture plus a shared logit of 1.5), restated with the
  lowest-index rule: [0, 1, 2, 3, 11, 35, 67, 99, 128];
- the shared weight against scipy's float64 `expit` rounded to float32, for logits of
  both signs (a planted mistake, the stable form's negative branch dropped, fails);
- the shared logit never enters the selection or the routed weights, however large;
- unnormalised weights against torch's float64 softmax of the whole row, summing below
  one, and equal to the renormalised weights times their own sum.

Sigmoid routing with a correction bias (route/ordinal.py:200-286):

- the ordinal map against float order itself (a stable sort of the floats), over
  random, signed-zero, subnormal, infinite and NaN keys;
- the float32 sigmoid against torch's float64 sigmoid rounded to float32;
- the reference's tie fixture (tests/test_kernel_router_ordinal.py:88-142): zero bias,
  k = 8 over 256 experts gives [0, 1, 2, 3, 11, 35, 67, 99];
- the reference's separated rows with a graded bias (test_kernel_router_ordinal.py:
  53-70): indices equal to a float64 chain's stable sort of score + bias, weights within
  1e-5 of its float64 renormalisation; the bias selects and never weighs;
- a brute force over rows with ties everywhere;
- the key permutation property of the fused router (test_kernel_residual_rms_router.py:
  139-171): the stable ascending order of the keys is the stable descending order of
  score + bias;
- planted mistakes (upward ties, the bias ignored, weights from the biased scores, no
  renormalisation, NaN first) fail.
"""

import numpy as np
import pytest
import torch

from oracle import route
from oracle.bf16 import from_float, to_f32, ulp_distance

KAT_EXPECTED = [0, 1, 2, 3, 11, 35, 67, 99]


def tied_logits(experts: int) -> np.ndarray:
    values = np.arange(experts, dtype=np.float64) * -0.5
    values[[3, 11, 35, 67, 99, 120]] = values[3]
    return from_float(values)[None, :]


@pytest.mark.parametrize("experts", [128, 256])
def test_reference_tie_fixture_lowest_index(experts):
    assert route.select(tied_logits(experts), 8)[0].tolist() == KAT_EXPECTED


def _brute(row_values, k, lower=True):
    order = sorted(range(len(row_values)), key=lambda e: (-row_values[e], e if lower else -e))
    return order[:k]


def test_upward_rule_brute_force_matches_reference_answer():
    values = to_f32(tied_logits(128))[0].tolist()
    assert _brute(values, 8, lower=False) == [0, 1, 2, 120, 99, 67, 35, 11]


def test_selection_matches_brute_force_and_torch():
    rng = np.random.default_rng(0)
    # Few distinct values, so ties are everywhere.
    logits = from_float(rng.integers(-6, 6, size=(200, 64)) * 0.25)
    got = route.select(logits, 8)
    values = to_f32(logits)
    for row in range(200):
        assert got[row].tolist() == _brute(values[row].tolist(), 8)
    torch_idx = torch.sort(torch.from_numpy(values), dim=-1, descending=True, stable=True).indices[:, :8]
    assert np.array_equal(got, torch_idx.numpy())


def test_weights_descend_sum_to_one_and_match_torch():
    rng = np.random.default_rng(1)
    logits = from_float(rng.standard_normal((300, 128)))
    idx, w = route.softmax_topk(logits, 8)
    assert (np.diff(w, axis=-1) <= 0).all()
    np.testing.assert_allclose(w.sum(-1), 1.0, atol=1e-6)
    p = torch.softmax(torch.from_numpy(to_f32(logits)).double(), -1)
    kept = torch.gather(p, -1, torch.from_numpy(idx.astype(np.int64)))
    np.testing.assert_allclose(w, (kept / kept.sum(-1, keepdim=True)).numpy(), rtol=2e-6)


def test_logits_agree_with_torch_bf16_matmul():
    rng = np.random.default_rng(2)
    n = from_float(rng.standard_normal((64, 2048)))
    wg = from_float(0.02 * rng.standard_normal((128, 2048)))
    got = route.router_logits(n, wg)
    t = lambda b: torch.from_numpy(b.view(np.int16)).view(torch.bfloat16)
    want = (t(n) @ t(wg).T).view(torch.int16).numpy().view(np.uint16)
    dist = ulp_distance(got, want)
    assert dist.max() <= 1 and np.mean(dist == 0) > 0.99


def test_signed_zero_ties_and_nan_last():
    row = np.array([[0x8000, 0x0000, 0x3F80, 0x7FC0, 0xBF80, 0xFF80]], np.uint16)  # -0, +0, 1, NaN, -1, -inf
    assert route.select(row, 6)[0].tolist() == [2, 0, 1, 4, 5, 3]


def test_planted_mistakes_fail():
    logits = tied_logits(128)
    keys = route.order_keys(logits)
    upward = np.argsort(keys[0], kind="stable")[::-1][:8]
    assert upward.tolist() != KAT_EXPECTED
    ascending = np.argsort(keys[0], kind="stable")[:8]
    assert ascending.tolist() != KAT_EXPECTED
    rng = np.random.default_rng(3)
    lg = from_float(rng.standard_normal((10, 128)))
    idx, w = route.softmax_topk(lg, 8)
    unnormalised = np.take_along_axis(
        torch.softmax(torch.from_numpy(to_f32(lg)), -1).numpy(), idx.astype(np.int64), -1)
    assert not np.allclose(unnormalised.sum(-1), 1.0, atol=1e-3)


# ---- sigmoid routing with a correction bias -----------------------------------------

EXPERTS = 256


def _f64_chain(logits_f32, bias, k):
    """The reference test's op chain (test_kernel_router_ordinal.py:39-50): float64
    scores and sum, stable descending sort, float64 renormalisation."""
    x = np.asarray(logits_f32, dtype=np.float64)
    y = 1.0 / (1.0 + np.exp(np.abs(x)))
    scores = np.where(x < 0.0, y, 1.0 - y)
    biased = scores + np.asarray(bias, dtype=np.float64)
    chosen = np.argsort(-biased, kind="stable", axis=-1)[:, :k]
    picked = np.take_along_axis(scores, chosen, axis=-1)
    return chosen, picked / picked.sum(axis=-1, keepdims=True)


def _separated(rows, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((rows, EXPERTS)) * 2.0).astype(np.float32)


def _graded_bias(logits_f32, seed):
    """score + bias on a permuted grid four apart (test_kernel_router_ordinal.py:58-70)."""
    rng = np.random.default_rng(seed)
    x = logits_f32[0].astype(np.float64)
    y = 1.0 / (1.0 + np.exp(np.abs(x)))
    scores = np.where(x < 0.0, y, 1.0 - y)
    grid = np.empty(EXPERTS)
    grid[rng.permutation(EXPERTS)] = (np.arange(EXPERTS) - EXPERTS / 2) * 4.0
    return (grid - scores).astype(np.float32)


def test_ordinal_follows_float_order():
    rng = np.random.default_rng(10)
    values = np.concatenate([
        rng.standard_normal(2000).astype(np.float32) * np.float32(10.0) ** rng.integers(-40, 38, 2000),
        np.array([0.0, -0.0, np.inf, -np.inf, 1e-45, -1e-45, 3.4e38, -3.4e38], np.float32),
    ]).astype(np.float32)
    keys = route.ordinal(values)
    order = np.argsort(keys, kind="stable")
    assert np.all(np.diff(values[order].astype(np.float64)) >= 0)
    assert route.ordinal(np.float32(0.0)) == route.ordinal(np.float32(-0.0)) == 0x80000000
    nan = route.ordinal(np.array([np.nan, -np.nan], np.float32))
    assert (nan == 0xFFFFFFFF).all() and (keys < 0xFFFFFFFF).all()
    # The reference's op form (ordinal.py:253-262, no NaN or zero arm) agrees off those.
    bits = values.view(np.uint32).astype(np.uint64)
    plain = np.where(bits & 0x80000000, (~bits) & 0xFFFFFFFF, bits ^ 0x80000000)
    finite_nonzero = np.isfinite(values) & (values != 0)
    assert np.array_equal(keys[finite_nonzero], plain[finite_nonzero].astype(np.uint32))


def test_sigmoid_f32_is_the_rounded_float64_sigmoid():
    rng = np.random.default_rng(11)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 8,
                        np.array([0.0, -0.0, 1e-30, 88.0, -88.0, 104.0, -104.0, np.inf, -np.inf],
                                 np.float32)]).astype(np.float32)
    want = torch.sigmoid(torch.from_numpy(x).double()).float().numpy()
    got = route.sigmoid_f32(x)
    assert np.array_equal(got, want)
    assert np.isnan(route.sigmoid_f32(np.array([np.nan], np.float32)))[0]


@pytest.mark.parametrize("as_bf16", [False, True])
def test_sigmoid_tie_fixture(as_bf16):
    values = np.arange(EXPERTS, dtype=np.float64) * -0.5
    values[[3, 11, 35, 67, 99, 120]] = values[3]
    logits = (to_f32(from_float(values)) if as_bf16 else values.astype(np.float32))[None, :]
    idx, w, _ = route.sigmoid_topk(logits, np.zeros(EXPERTS, np.float32), 8)
    assert idx[0].tolist() == KAT_EXPECTED
    assert (np.diff(w[0]) <= 0).all() and abs(float(w[0].sum()) - 1.0) < 1e-6


@pytest.mark.parametrize("rows", [1, 5])
def test_sigmoid_matches_the_float64_chain_on_separated_rows(rows):
    for seed in range(4):
        logits = _separated(rows, seed)
        bias = _graded_bias(logits, seed + 100)
        idx, w, _ = route.sigmoid_topk(logits, bias, 8)
        ref_idx, ref_w = _f64_chain(logits, bias, 8)
        assert idx.tolist() == ref_idx.tolist()
        assert np.abs(w - ref_w).max() / np.abs(ref_w).max() < 1e-5


def test_bias_selects_but_never_weighs():
    logits = _separated(1, 3)
    bias = _graded_bias(logits, 300)
    base, _, _ = route.sigmoid_topk(logits, bias, 8)
    outsider = next(e for e in range(EXPERTS) if e not in set(base[0].tolist()))
    boosted = bias + np.where(np.arange(EXPERTS) == outsider, 1e4, 0.0).astype(np.float32)
    idx, w, _ = route.sigmoid_topk(logits, boosted, 8)
    ref_idx, ref_w = _f64_chain(logits, boosted, 8)
    assert idx[0][0] == outsider and idx.tolist() == ref_idx.tolist()
    assert np.abs(w - ref_w).max() < 1e-5


def test_sigmoid_selection_brute_force_with_ties():
    rng = np.random.default_rng(12)
    logits = (rng.integers(-4, 4, size=(300, 64)) * 0.5).astype(np.float32)
    bias = (rng.integers(-2, 2, size=64) * 0.25).astype(np.float32)
    idx, w, keys = route.sigmoid_topk(logits, bias, 6)
    scores = route.sigmoid_f32(logits)
    biased = (scores + bias).astype(np.float32)
    for row in range(300):
        order = sorted(range(64), key=lambda e: (-float(biased[row, e]), e))[:6]
        assert idx[row].tolist() == order
        total = np.float32(0)
        for e in order:
            total = np.float32(scores[row, e] + total)
        assert np.array_equal(w[row], (scores[row, order] / total).astype(np.float32))


def test_nan_scores_rank_last():
    logits = np.array([[1.0, np.nan, -1.0, 0.0]], np.float32)
    idx, _, keys = route.sigmoid_topk(logits, np.zeros(4, np.float32), 4)
    assert idx[0].tolist() == [0, 3, 2, 1] and keys[0][1] == 0xFFFFFFFF


def test_key_permutation_property_of_the_fused_router():
    rng = np.random.default_rng(13)
    hidden, experts = 512, 64
    x = from_float(rng.standard_normal((1, hidden)))
    r = from_float(rng.standard_normal((1, hidden)))
    w = from_float(1 + 0.1 * rng.standard_normal(hidden))
    wg = from_float(rng.standard_normal((experts, hidden)) * hidden ** -0.5)
    zero = np.zeros(experts, np.float32)
    _, _, logits, _, _, _ = route.residual_rms_router_sigmoid(x, r, w, wg, zero, 1e-6, 8)
    x64 = to_f32(logits)[0].astype(np.float64)
    scores = np.where(x64 < 0, 1 / (1 + np.exp(np.abs(x64))), 1 - 1 / (1 + np.exp(np.abs(x64))))
    grid = np.empty(experts)
    grid[rng.permutation(experts)] = (np.arange(experts) - experts / 2) * 4.0
    bias = (grid - scores).astype(np.float32)
    _, _, again, keys, idx, _ = route.residual_rms_router_sigmoid(x, r, w, wg, bias, 1e-6, 8)
    assert np.array_equal(again, logits)
    expected = np.argsort(-(scores + bias.astype(np.float64)), kind="stable")
    assert np.argsort(keys[0], kind="stable").tolist() == expected.tolist()
    assert idx[0].tolist() == expected[:8].tolist()


def test_sigmoid_planted_mistakes_fail():
    values = np.arange(EXPERTS, dtype=np.float64) * -0.5
    values[[3, 11, 35, 67, 99, 120]] = values[3]
    logits = values.astype(np.float32)[None, :]
    zero = np.zeros(EXPERTS, np.float32)
    _, keys = route.sigmoid_keys(logits, zero)
    upward = np.argsort(keys[0].astype(np.int64) * 1024 - np.arange(EXPERTS))[:8]
    assert upward.tolist() != KAT_EXPECTED
    sep = _separated(2, 5)
    bias = _graded_bias(sep, 105)
    ref_idx, ref_w = _f64_chain(sep, bias, 8)
    no_bias, _, _ = route.sigmoid_topk(sep, zero, 8)
    assert no_bias.tolist() != ref_idx.tolist()
    scores = route.sigmoid_f32(sep)
    biased = (scores + bias).astype(np.float32)
    from_biased = np.take_along_axis(biased, ref_idx, -1)
    assert not np.allclose(from_biased / from_biased.sum(-1, keepdims=True), ref_w, atol=1e-3)
    unnormalised = np.take_along_axis(scores, ref_idx, -1)
    assert not np.allclose(unnormalised, ref_w, atol=1e-3)
    nan_first = np.argsort(np.where(np.isnan(np.array([1.0, np.nan], np.float32)), 0, 1))
    assert nan_first.tolist() != route.sigmoid_topk(np.array([[1.0, np.nan]], np.float32),
                                                    np.zeros(2, np.float32), 2)[0][0].tolist()


# ---- the shared slot and normalize=False --------------------------------------------


def test_reference_shared_slot_fixture_lowest_index():
    logits = np.concatenate([tied_logits(128), from_float(np.array([[1.5]]))], axis=-1)
    idx, w = route.softmax_topk_slots(logits, 8, shared=True)
    assert idx[0].tolist() == KAT_EXPECTED + [128]
    assert w[0, 8] == np.float32(1.0 - 1.0 / (1.0 + np.exp(1.5)))
    routed_idx, routed_w = route.softmax_topk(tied_logits(128), 8)
    assert np.array_equal(idx[:, :8], routed_idx) and np.array_equal(w[:, :8], routed_w)


def test_shared_weight_is_the_rounded_sigmoid_on_both_sides():
    from scipy.special import expit

    rng = np.random.default_rng(21)
    gate = from_float(np.concatenate([rng.standard_normal(400) * 6, [0.0, -0.0, 30.0, -30.0, 90.0, -90.0]]))
    logits = np.concatenate([from_float(rng.standard_normal((gate.size, 64))), gate[:, None]], axis=-1)
    _, w = route.softmax_topk_slots(logits, 4, shared=True)
    want = expit(to_f32(gate).astype(np.float64)).astype(np.float32)
    assert np.array_equal(w[:, 4], want)
    negative = to_f32(gate) < 0
    assert (w[negative, 4] < 0.5).all() and (w[~negative, 4] >= 0.5).all()
    # planted: the stable form without its negative branch (y for every sign)
    x = to_f32(gate).astype(np.float64)
    dropped = (1.0 / (1.0 + np.exp(np.abs(x)))).astype(np.float32)
    assert not np.array_equal(dropped, w[:, 4])


def test_shared_logit_never_selects_or_weighs_the_routed_slots():
    rng = np.random.default_rng(22)
    routed = from_float(rng.standard_normal((50, 128)))
    base_idx, base_w = route.softmax_topk_slots(routed, 8)
    for value in (-80.0, 0.0, 3.0, 80.0):
        logits = np.concatenate([routed, from_float(np.full((50, 1), value))], axis=-1)
        for normalize in (True, False):
            idx, w = route.softmax_topk_slots(logits, 8, normalize=normalize, shared=True)
            want_idx, want_w = route.softmax_topk_slots(routed, 8, normalize=normalize)
            assert np.array_equal(idx[:, :8], want_idx) and np.array_equal(w[:, :8], want_w)
            assert (idx[:, 8] == 128).all()
    assert np.array_equal(base_idx, route.select(routed, 8))


def test_unnormalised_weights_are_the_row_probabilities():
    rng = np.random.default_rng(23)
    logits = from_float(rng.standard_normal((300, 128)) * 2)
    idx, w = route.softmax_topk_slots(logits, 8, normalize=False)
    assert np.array_equal(idx, route.select(logits, 8))
    p = torch.softmax(torch.from_numpy(to_f32(logits)).double(), -1)
    want = torch.gather(p, -1, torch.from_numpy(idx.astype(np.int64))).numpy()
    np.testing.assert_allclose(w, want, rtol=2e-6)
    assert (w.sum(-1) < 1.0).all() and (np.diff(w, axis=-1) <= 0).all()
    _, renormalised = route.softmax_topk_slots(logits, 8)
    np.testing.assert_allclose(renormalised, w / w.sum(-1, keepdims=True), rtol=2e-6)
    # planted: renormalising anyway is a different answer
    assert not np.allclose(renormalised, w, rtol=1e-3)

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
- -0 and +0 tie; NaN sorts above everything;
- planted mistakes (upward ties, no renormalisation, ascending order) fail.
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


def test_signed_zero_ties_and_nan_first():
    row = np.array([[0x8000, 0x0000, 0x3F80, 0x7FC0, 0xBF80]], np.uint16)  # -0, +0, 1, NaN, -1
    assert route.select(row, 5)[0].tolist() == [3, 2, 0, 1, 4]


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

"""Pins the routing oracle (`oracle/routing.py`) against the reference's own
known answers and against independent computations (torch.topk, brute-force
subset enumeration). CPU only."""

import itertools

import numpy as np
import pytest
import torch

from oracle import routing

EXPERTS, TOPK = 512, 10  # `tests/kernels/test_router_topk.py:30-31`


def test_rowmax_matches_torch_topk_on_softmax_scores():
    """`tests/kernels/test_router_topk.py:63-74`: values bit-identical to
    torch.topk, and the chosen ids gather exactly those values."""
    rng = np.random.default_rng(99)
    logits = torch.from_numpy(rng.standard_normal((1024, EXPERTS), dtype=np.float32) * 2.0).to(torch.bfloat16)
    scores = logits.float().softmax(dim=-1)
    kw, ki = routing.rowmax_topk(scores.numpy(), TOPK)
    ref_v, _ = torch.topk(scores, TOPK, dim=-1)
    np.testing.assert_array_equal(kw, ref_v.numpy())
    gathered = torch.gather(scores, 1, torch.from_numpy(ki).long())
    np.testing.assert_array_equal(gathered.numpy(), ref_v.numpy())


def test_all_nan_row_selects_k_distinct_experts():
    """`test_router_topk.py:77-97`."""
    kw, ki = routing.rowmax_topk(np.full((3, EXPERTS), np.nan, np.float32), TOPK)
    assert np.isnan(kw).all()
    for row in ki:
        assert sorted(row.tolist()) == list(range(TOPK))


def test_partial_nan_row_selects_k_distinct_finite_experts():
    """`test_router_topk.py:100-108`."""
    rng = np.random.default_rng(5)
    scores = rng.random((2, EXPERTS), dtype=np.float32)
    scores[:, :5] = np.nan
    kw, ki = routing.rowmax_topk(scores, TOPK)
    assert np.isfinite(kw).all()
    for row in ki:
        assert len(set(row.tolist())) == TOPK and min(row.tolist()) >= 5


@pytest.mark.parametrize("bad", [np.nan, -np.inf, np.finfo(np.float32).min])
def test_row_at_or_below_sentinel(bad):
    """`test_router_topk.py:111-135`: NaN weights, ids exactly 0..k-1."""
    kw, ki = routing.rowmax_topk(np.full((3, EXPERTS), bad, np.float32), TOPK)
    assert np.isnan(kw).all()
    for row in ki:
        assert row.tolist() == list(range(TOPK))


def test_ties_and_nan_table():
    """`test_router_topk.py:138-150`, with the answers written out."""
    s = np.zeros((4, EXPERTS), np.float32)
    s[0] = 1.0 / EXPERTS
    s[1, 200:212] = 4.0
    s[2] = np.nan
    s[3, :3] = np.nan
    s[3, 300:310] = np.linspace(1.0, 0.1, 10)
    kw, ki = routing.rowmax_topk(s, TOPK)
    assert ki[0].tolist() == list(range(10))  # all tied -> lowest ids
    assert ki[1].tolist() == list(range(200, 210))  # tie across the k boundary
    assert np.isnan(kw[2]).all() and ki[2].tolist() == list(range(10))
    assert ki[3].tolist() == list(range(300, 310))
    np.testing.assert_array_equal(kw[3], np.linspace(1.0, 0.1, 10).astype(np.float32))
    np.testing.assert_array_equal(kw[0], np.full(10, 1.0 / EXPERTS, np.float32))


def test_routed_scaling_factor_known_answer():
    """`tests/layers/adapter/test_moe_routing.py:222-234`; plus the closed
    form of softmax top-2 renormalized: e^4/(e^4+e^3), e^3/(e^4+e^3)."""
    logits = np.array([[1.0, 2.0, 3.0, 4.0], [4.0, 3.0, 2.0, 1.0]], np.float32)
    w1, i1 = routing.select_experts(logits, 2, True, "softmax")
    w2, i2 = routing.select_experts(logits, 2, True, "softmax", routed_scaling_factor=2.5)
    assert i1.tolist() == [[3, 2], [0, 1]]
    np.testing.assert_array_equal(i1, i2)
    a = np.exp(4.0) / (np.exp(4.0) + np.exp(3.0))
    np.testing.assert_allclose(w1, [[a, 1 - a], [a, 1 - a]], rtol=4e-3)  # bf16 weights
    np.testing.assert_allclose(w2, w1 * 2.5, rtol=4e-3)


def test_uniform_scores_give_equal_weights():
    """Uniform logits: every expert scores 1/E (`test_moe_routing.py:237-251`
    uses this to isolate the scaling factor); without renormalization each
    weight is the score times the factor."""
    w, ids = routing.select_experts(np.zeros((2, 4), np.float32), 2, False, "softmax",
                                    routed_scaling_factor=2.0)
    assert ids.tolist() == [[0, 1], [0, 1]]
    np.testing.assert_array_equal(w, np.full((2, 2), 0.5, np.float32))


def test_bias_chooses_but_does_not_weight():
    """`moe_routing.py:306-311`: the bias changes which experts are chosen;
    the weights are the unbiased scores at those experts."""
    logits = np.array([[0.0, 1.0, 2.0, 3.0]], np.float32)
    bias = np.array([10.0, 0.0, 0.0, 0.0], np.float32)
    w, ids = routing.select_experts(logits, 2, False, "sigmoid", bias)
    assert ids.tolist() == [[0, 3]]
    np.testing.assert_allclose(w[0], [1 / (1 + np.exp(-0.0)), 1 / (1 + np.exp(-3.0))], rtol=4e-3)


def _brute_grouped(c, s, k, g, kg):
    """Exhaustive form of the grouped rule for one token: the best set of kg
    groups by summed group score, then the best k-subset of their experts by
    summed choice score, returned in descending choice order."""
    e = c.shape[0]
    per = e // g
    gscore = [np.sort(c[j * per:(j + 1) * per])[-2:].sum() for j in range(g)]
    best_groups = max(itertools.combinations(range(g), kg), key=lambda gs: sum(gscore[j] for j in gs))
    pool = [x for j in best_groups for x in range(j * per, (j + 1) * per)]
    best = max(itertools.combinations(pool, k), key=lambda xs: sum(float(c[x]) for x in xs))
    ids = sorted(best, key=lambda x: -c[x])
    return ids


@pytest.mark.parametrize("seed", range(6))
def test_grouped_topk_matches_exhaustive_search(seed):
    """The build's grouped rule (parity with upstream vLLM unpinned) checked
    against a subset enumeration on 16 experts / 4 groups / 2 kept / top-4."""
    rng = np.random.default_rng(seed)
    T, E, G, KG, K = 5, 16, 4, 2, 4
    logits = rng.standard_normal((T, E)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    w, ids = routing.grouped_topk(logits, K, True, G, KG, "sigmoid", bias, 2.5)
    s = routing.scores_of(logits, "sigmoid")
    c = (s + bias[None, :]).astype(np.float32)
    for t in range(T):
        assert ids[t].tolist() == _brute_grouped(c[t], s[t], K, G, KG)
        sw = s[t, ids[t]]
        np.testing.assert_allclose(w[t], sw / sw.sum() * 2.5, rtol=4e-3)


def test_grouped_with_all_groups_kept_is_plain_biased_topk():
    """Keeping every group reduces the grouped rule to the plain biased top-k."""
    rng = np.random.default_rng(1)
    logits = rng.standard_normal((7, 32)).astype(np.float32)
    bias = (rng.standard_normal(32) * 0.1).astype(np.float32)
    wg, ig = routing.grouped_topk(logits, 6, True, 4, 4, "sigmoid", bias, 1.0)
    wp, ip = routing.select_experts(logits, 6, True, "sigmoid", bias)
    np.testing.assert_array_equal(ig, ip)
    np.testing.assert_array_equal(wg, wp)


def test_hash_select_known_answer():
    """`tests/layers/adapter/test_moe_routing.py:237-251`: uniform logits
    score every one of 4 experts 0.25; ids come from the table rows of the
    input ids; without renormalization the factor 2.0 alone shapes the
    weights."""
    logits = np.zeros((2, 4), np.float32)
    w, ids = routing.hash_select(logits, [[0, 1], [2, 3]], [1, 0], False, "softmax", 2.0)
    assert ids.tolist() == [[2, 3], [0, 1]]
    np.testing.assert_array_equal(w, np.full((2, 2), 0.5, np.float32))


def test_hash_select_gathers_unbiased_scores_and_renormalizes():
    rng = np.random.default_rng(4)
    logits = rng.standard_normal((5, 16)).astype(np.float32)
    table = rng.integers(0, 16, (7, 3))
    inp = np.array([6, 0, 3, 3, 1])
    w, ids = routing.hash_select(logits, table, inp, True, "sigmoid", 1.5)
    s = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    exp_ids = table[inp]
    g = np.take_along_axis(s, exp_ids, axis=-1)
    np.testing.assert_array_equal(ids, exp_ids)
    np.testing.assert_allclose(w, g / g.sum(-1, keepdims=True) * 1.5, rtol=8e-3)

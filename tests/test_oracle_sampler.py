"""Pins the sampling oracle (oracle/sampler.py) with hand-computed cases and
brute force on tiny vocabularies."""

import itertools
import math

import torch

from oracle import sampler as osm


def L(*v):
    return torch.tensor(v, dtype=torch.float64)


def test_single_rule_keeps_crossing_token_batch_rule_does_not():
    # probs 0.5, 0.3, 0.2 (log-space), p = 0.6: cumsum 0.5, 0.8, 1.0
    x = torch.log(L(0.2, 0.5, 0.3))
    single = osm.distribution(x, top_p=0.6, rule=osm.RULE_SINGLE)
    batch = osm.distribution(x, top_p=0.6, rule=osm.RULE_BATCH)
    assert torch.allclose(single, L(0.0, 0.5 / 0.8, 0.3 / 0.8))
    assert torch.allclose(batch, L(0.0, 1.0, 0.0))
    # p below the top probability: both keep exactly the top token
    for rule in (osm.RULE_SINGLE, osm.RULE_BATCH):
        assert torch.allclose(osm.distribution(x, top_p=0.4, rule=rule), L(0.0, 1.0, 0.0))


def test_top_k_then_top_p_batch_rule():
    x = torch.log(L(0.4, 0.3, 0.2, 0.1))
    # top_k = 3 renormalises to 4/9, 3/9, 2/9; p = 0.8 keeps cumsum 4/9, 7/9 (<= 0.8)
    d = osm.distribution(x, top_k=3, top_p=0.8, rule=osm.RULE_BATCH)
    assert torch.allclose(d, L(4 / 7, 3 / 7, 0.0, 0.0))
    # the single rule ignores top_p when top_k is set
    d = osm.distribution(x, top_k=3, top_p=0.8, rule=osm.RULE_SINGLE)
    assert torch.allclose(d, L(4 / 9, 3 / 9, 2 / 9, 0.0))


def test_temperature_ban_and_bias():
    x = L(1.0, 2.0, 3.0, 9.0)
    d = osm.distribution(x, temperature=0.5, max_valid_id=2)
    e = torch.exp(L(2.0, 4.0, 6.0))
    assert torch.allclose(d[:3], e / e.sum()) and d[3] == 0
    d = osm.distribution(x, logit_bias={"0": 500.0})  # clamped to +100
    assert d[0] > 0.999999
    # the clamp itself: equal logits with biases +150 and +100 both reach +100,
    # so the two tokens stay equiprobable (unclamped, token 0 would take ~all)
    for rule in (osm.RULE_BATCH, osm.RULE_SINGLE):
        d = osm.distribution(L(0.0, 0.0, 0.0), logit_bias={"0": 150.0, "1": 100.0, "2": -250.0}, rule=rule)
        assert torch.allclose(d, L(0.5, 0.5, 0.0))
        d = osm.distribution(L(0.0, 0.0, 0.0), logit_bias={"0": -150.0, "1": -100.0}, rule=rule)
        assert torch.allclose(d, L(0.0, 0.0, 1.0))
        # below the clamp a bias is added as given
        d = osm.distribution(L(0.0, 0.0, 0.0), logit_bias={"0": math.log(3.0)}, rule=rule)
        assert torch.allclose(d, L(0.6, 0.2, 0.2))
    assert osm.greedy(x, max_valid_id=2)[0] == 2
    t, lp = osm.greedy(L(1.0, 5.0, 5.0))
    assert t == 1 and math.isclose(lp, math.log(math.exp(5) / (math.exp(1) + 2 * math.exp(5))))


def test_nucleus_brute_force():
    g = torch.Generator().manual_seed(0)
    for _ in range(200):
        V = 5
        x = torch.randn(V, generator=g, dtype=torch.float64) * 2
        p = float(torch.rand(1, generator=g))
        probs = torch.softmax(x, -1)
        order = sorted(range(V), key=lambda i: (-float(x[i]), i))
        # batch rule: longest prefix with cumulative mass <= p (at least one)
        n = 0
        acc = 0.0
        for i in order:
            acc += float(probs[i])
            if acc <= p:
                n += 1
        n_batch = max(1, n)
        n_single = n + 1
        for rule, m in ((osm.RULE_BATCH, n_batch), (osm.RULE_SINGLE, n_single)):
            d = osm.distribution(x, top_p=p, rule=rule)
            kept = set(order[:m])
            assert {i for i in range(V) if d[i] > 0} == kept
            assert math.isclose(float(d.sum()), 1.0, rel_tol=1e-12)


def test_repetition_penalty_per_occurrence():
    x = torch.tensor([[2.0, -2.0, 1.0]])
    out = osm.repetition_penalty(x, [[0, 0, 1, 5]], 2.0)
    assert torch.allclose(out, torch.tensor([[0.5, -4.0, 1.0]], dtype=torch.float64))


def test_generate_rule_top_k_then_nucleus_keeping_crossing():
    """generation_mixin.py:188-211 by hand: probs 0.4, 0.3, 0.2, 0.1.
    top_k = 3 -> 4/9, 3/9, 2/9; top_p = 0.5 keeps 4/9 (cum 4/9 <= .5) and the
    crossing 3/9 -> 4/7, 3/7.  top_p = 0 (or 1) applies no nucleus at all; top_k
    = 0 with top_p = 0.65 keeps .4, .3 (cum before .3 is .4 <= .65) and .2 (cum
    before is .7 > .65 -> removed): 4/7, 3/7."""
    x = torch.log(L(0.4, 0.3, 0.2, 0.1))
    d = osm.distribution(x, top_k=3, top_p=0.5, rule=osm.RULE_MIXIN)
    assert torch.allclose(d, L(4 / 7, 3 / 7, 0.0, 0.0))
    for p in (0.0, 1.0):
        d = osm.distribution(x, top_k=3, top_p=p, rule=osm.RULE_MIXIN)
        assert torch.allclose(d, L(4 / 9, 3 / 9, 2 / 9, 0.0))
    d = osm.distribution(x, top_k=0, top_p=0.65, rule=osm.RULE_MIXIN)
    assert torch.allclose(d, L(4 / 7, 3 / 7, 0.0, 0.0))
    # no filter: the softmax itself
    assert torch.allclose(osm.distribution(x, rule=osm.RULE_MIXIN), L(0.4, 0.3, 0.2, 0.1))
    # temperature 0.5 squares and renormalises the probabilities
    d = osm.distribution(x, temperature=0.5, rule=osm.RULE_MIXIN)
    q = L(0.16, 0.09, 0.04, 0.01)
    assert torch.allclose(d, q / q.sum())


def test_non_finite_probabilities_fall_back_to_uniform():
    """TokenSampler.sample (core.py:102-108): a softmax holding NaN or inf, from a
    NaN logit, a +inf logit or a row of -inf, is replaced by the uniform
    distribution over the vocabulary, before top-k / top-p (whose ties then keep
    every token)."""
    V = 6
    rows = [L(1.0, float("nan"), 2.0, 0.0, 0.0, 0.0),
            L(1.0, float("inf"), 2.0, 0.0, 0.0, 0.0),
            torch.full((V,), float("-inf"), dtype=torch.float64)]
    for x in rows:
        for kw in ({}, {"top_p": 0.5}, {"top_k": 2}):
            d = osm.distribution(x, rule=osm.RULE_SINGLE, **kw)
            assert torch.allclose(d, torch.full((V,), 1.0 / V, dtype=torch.float64)), (x, kw)
    # a finite row keeps its softmax
    d = osm.distribution(L(0.0, math.log(2.0), 0.0), rule=osm.RULE_SINGLE)
    assert torch.allclose(d, L(0.25, 0.5, 0.25))

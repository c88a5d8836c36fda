"""Pins for the oracle's policy restatement (CPU): the reference's known
answers and mode checks, Python's stable sorted on random/tied inputs, and
the fixed-order block mass against float64 sums."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import COLD_STATE, HOT_STATE, WARM_STATE
from oracle import policy as P


def test_known_answer_block_scores_and_budget():
    # main.py:375-389
    pattern = np.concatenate([np.full(16, v, np.float16) for v in (0.4, 0.9, 0.1, 0.2)])
    attn = np.tile(pattern.reshape(1, 1, 1, 64), (1, 32, 1, 1))
    scores = P.compute_block_scores(attn, 16)
    np.testing.assert_allclose(scores, [0.4, 0.9, 0.1, 0.2], rtol=1e-3)
    assert P.enforce_budget(list(scores), [0, 0, 0, 0], hot_budget=3) == [0, 0, 1, 0]


def test_policy_modes_match_reference_checks():
    # main.py:700-719 with scores arange(12)
    scores = list(np.arange(12, dtype=np.float32))
    cur = [HOT_STATE] * 12
    assert set(P.tier_labels(np.array([scores]), np.array([cur]), 4, 2, "hot_only")[0]) == {HOT_STATE}
    assert WARM_STATE in set(P.enforce_budget(scores, cur, 4))
    tiered = set(P.enforce_tiered_budget(scores, cur, 4, 2))
    assert WARM_STATE in tiered and COLD_STATE in tiered


def _sorted_reference(scores, n, hot_budget, warm_budget):
    """Independent statement via Python's stable sort on (-score, index)."""
    cands = [i for i in range(n) if i not in (0, n - 1)]
    ranked = sorted(cands, key=lambda i: (-float(scores[i]), i))
    extra = max(hot_budget - 2, 0)
    return set(ranked[:extra]), set(ranked[extra: extra + max(warm_budget, 0)])


def test_tiered_budget_matches_stable_sort_with_ties():
    rng = np.random.default_rng(0)
    for trial in range(300):
        n = int(rng.integers(3, 40))
        scores = (rng.integers(0, 5, n) * 0.5).astype(np.float32) if trial % 2 else rng.standard_normal(n)
        hot, warm = int(rng.integers(0, n + 2)), int(rng.integers(0, n + 2))
        cur = rng.integers(0, 3, n).tolist()
        got = P.enforce_tiered_budget(list(scores), cur, hot, warm)
        hs, ws = _sorted_reference(scores, n, hot, warm)
        for i in range(n):
            want = HOT_STATE if i in (0, n - 1) or i in hs else (WARM_STATE if i in ws else COLD_STATE)
            if cur[i] == COLD_STATE:
                want = COLD_STATE
            assert got[i] == want


def test_small_sequences_are_all_hot_even_from_cold():
    # n <= 2 promotes every block to HOT (tierkv_policy.py:1413-1417)
    assert P.enforce_budget([0.1, 0.2], [2, 1], 0) == [0, 0]
    assert P.enforce_tiered_budget([0.1], [2], 0, 0) == [0]


def test_prefill_states_modes():
    s = np.array([1.0, 0.2, 0.9, 0.1, 0.5, 1.0], np.float32)
    assert P.desired_prefill_states(6, s, 3, 1, "hot_warm") == [0, 1, 0, 1, 1, 0]
    assert P.desired_prefill_states(6, s, 3, 1, "hot_warm_cold") == [0, 2, 0, 2, 1, 0]
    assert P.desired_prefill_states(6, s, 3, 1, "hot_only") == [0] * 6


def test_block_mass_order_and_value():
    rng = np.random.default_rng(1)
    logits = rng.standard_normal((2, 4, 128)).astype(np.float32) * 3
    probs = np.exp(logits) / np.exp(logits).sum(-1, keepdims=True)
    probs = probs.astype(np.float32)
    m = P.block_mass_from_probs(probs, 16)
    exact = probs.astype(np.float64).sum(1).reshape(2, 8, 16).sum(-1) / 4 / 16
    np.testing.assert_allclose(m, exact, rtol=1e-6)
    # the explicit order: heads sequential, tokens pairwise
    tok = np.zeros((2, 128), np.float32)
    for h in range(4):
        tok = tok + probs[:, h]
    blk = tok.reshape(2, 8, 16)
    pair = [((((b[0] + b[1]) + (b[2] + b[3])) + ((b[4] + b[5]) + (b[6] + b[7])))
             + (((b[8] + b[9]) + (b[10] + b[11])) + ((b[12] + b[13]) + (b[14] + b[15]))))
            for b in blk.reshape(-1, 16)]
    want = (np.array(pair, np.float32).reshape(2, 8) / np.float32(4)) / np.float32(16)
    assert np.array_equal(m.view(np.uint32), want.astype(np.float32).view(np.uint32))


def test_scores_from_probability_sums():
    sums = np.array([[0.5, 0.25, 0.25, 0.0], [0.3, 0.3, 0.4, 0.0]], np.float32)
    got = P.block_scores_from_probability_sums(sums, np.array([16, 8, 0, 0]), 3)
    np.testing.assert_allclose(got, [0.4 / 16, 0.275 / 8, 0.325 / 1])


def test_bad_inputs_raise():
    with pytest.raises(ValueError):
        P.enforce_budget([0.1, 0.2, 0.3], [0, 0, 0], 2, demoted_state=0)
    with pytest.raises(ValueError):
        P.enforce_tiered_budget([0.1, 0.2], [0, 0, 0], 2, 1)


def test_prefill_block_mass_closed_forms():
    """oracle.policy.prefill_block_mass against what the mathematics fixes:
    with all keys zero every query spreads its probability uniformly over the
    keys it may see, p[q, t] = 1 / (q + 1) for t <= q, so the mass of token t
    is sum_{q >= t} 1 / (q + 1) / T; with one token the mass is 1; masses
    weighted by block length sum to 1 (every query row sums to 1)."""
    import numpy as np
    from oracle.policy import prefill_block_mass

    T, bs = 37, 16
    rng = np.random.default_rng(0)
    q = rng.standard_normal((1, 4, T, 8))
    k = np.zeros((1, 2, T, 8))
    got = prefill_block_mass(q, k, 0.3, bs)[0]
    per_token = np.array([sum(1.0 / (qq + 1) for qq in range(t, T)) / T for t in range(T)])
    want = [per_token[i * bs:(i + 1) * bs].mean() for i in range(-(-T // bs))]
    np.testing.assert_allclose(got, want, rtol=1e-12)
    assert prefill_block_mass(q[:, :, :1], k[:, :, :1], 0.3, bs)[0].tolist() == [1.0]
    k2 = rng.standard_normal((2, 2, T, 8))
    q2 = rng.standard_normal((2, 4, T, 8))
    m = prefill_block_mass(q2, k2, 0.5, bs)
    lens = np.array([min(bs, T - i * bs) for i in range(m.shape[1])])
    np.testing.assert_allclose((m * lens).sum(axis=1), 1.0, rtol=1e-12)
    # A key that dominates every logit takes (almost) all the mass of the
    # queries that can see it.
    k3 = np.zeros((1, 1, T, 8))
    k3[0, 0, 0] = 50.0
    q3 = np.ones((1, 1, T, 8))
    m3 = prefill_block_mass(q3, k3, 1.0, bs)[0]
    assert m3[0] * bs > 0.999

"""Property tests of the oracle itself (CPU, hypothesis, derandomized): facts
the mathematics fixes, checked over random inputs, so that a plausible slip
in the restatement (a wrong index, a dropped term, a transposed operand)
fails here and not only in a GPU comparison.

* absmax codec: codes in [-127, 127], the extreme code is +-127 whenever the
  tile is non-zero, and every value is reproduced within half a step;
* reference codec: codes in [0, 255] and every value reproduced within about
  one step (its fp16 op sequence rounds twice);
* decode: relabelling the physical slots (and moving the pool contents with
  them) leaves outputs and per-block probability sums unchanged, and a
  sequence whose blocks are all HOT equals dense softmax attention over its
  tokens;
* labels: the tier counts are fixed by the budgets (reserved first and last
  blocks, HOT budget, WARM budget, the rest COLD; sticky COLD aside)."""

from __future__ import annotations

import numpy as np
import pytest

hypothesis = pytest.importorskip("hypothesis")
from hypothesis import given, settings, strategies as st  # noqa: E402
from hypothesis.extra import numpy as hnp  # noqa: E402

from oracle import codec, policy  # noqa: E402
from oracle import decode as odecode  # noqa: E402

SETTINGS = dict(max_examples=60, deadline=None, derandomize=True, database=None)
f16_values = st.floats(-60000.0, 60000.0, allow_nan=False, allow_infinity=False, width=16)


@settings(**SETTINGS)
@given(hnp.arrays(np.float16, st.tuples(st.integers(1, 3), st.integers(1, 16), st.integers(1, 64)),
                  elements=f16_values))
def test_absmax_codec_bounds(x):
    q, s = codec.quantize_absmax_i8(x)
    assert q.dtype == np.int8 and q.min() >= -127 and q.max() <= 127
    xf = x.astype(np.float32)
    amax = np.abs(xf).max(axis=(-2, -1))
    assert (np.abs(q.astype(np.int32)).max(axis=(-2, -1))[amax > 0] == 127).all()
    deq = codec.dequantize_absmax_i8(q, s)
    step = s[..., None, None]
    assert (np.abs(deq - xf) <= 0.5 * step * (1 + 1e-6) + 1e-30).all()


@settings(**SETTINGS)
@given(hnp.arrays(np.float16, st.tuples(st.integers(1, 4), st.integers(2, 64)),
                  elements=st.floats(-100.0, 100.0, allow_nan=False, width=16)))
def test_reference_codec_bounds(x):
    q, s, z = codec.quantize_ref_u8(x)
    assert q.dtype == np.uint8
    deq = codec.dequantize_ref_u8(q, s, z).astype(np.float64)
    step = s.astype(np.float64)
    span = x.astype(np.float64).max(-1, keepdims=True) - x.astype(np.float64).min(-1, keepdims=True)
    # Within about one step plus the fp16 rounding of the values involved.
    tol = 1.01 * step + 2.0 ** -10 * (np.abs(x.astype(np.float64)) + span)
    assert (np.abs(deq - x) <= tol).all()


def _compact_case(rng, nb, n_hot, n_warm, kv, D, bs=16):
    states = np.full(nb, 2, np.int32)
    order = rng.permutation(nb)
    states[order[:n_hot]] = 0
    states[order[n_hot:n_hot + n_warm]] = 1
    table = np.full(nb, -1, np.int32)
    table[states == 0] = rng.permutation(n_hot)
    table[states == 1] = rng.permutation(n_warm)
    lengths = rng.integers(1, bs + 1, nb).astype(np.int32)
    hot_k = rng.standard_normal((max(n_hot, 1), kv, bs, D)).astype(np.float16)
    hot_v = rng.standard_normal((max(n_hot, 1), kv, bs, D)).astype(np.float16)
    wk, sk = codec.quantize_absmax_i8(rng.standard_normal((max(n_warm, 1), kv, bs, D)).astype(np.float16))
    wv, sv = codec.quantize_absmax_i8(rng.standard_normal((max(n_warm, 1), kv, bs, D)).astype(np.float16))
    return states, table, lengths, hot_k, hot_v, wk, wv, sk, sv


@settings(**SETTINGS)
@given(st.integers(0, 2 ** 31 - 1), st.integers(1, 24), st.sampled_from([1, 2]), st.sampled_from([1, 4]),
       st.sampled_from(["masked", "zero_logit"]))
def test_decode_invariant_under_slot_relabelling(seed, nb, kv, groups, cold):
    rng = np.random.default_rng(seed)
    n_hot = int(rng.integers(0, nb + 1))
    n_warm = int(rng.integers(0, nb - n_hot + 1))
    D = 16
    states, table, lengths, hk, hv, wk, wv, sk, sv = _compact_case(rng, nb, n_hot, n_warm, kv, D)
    q = rng.standard_normal((1, kv * groups, D)).astype(np.float16)
    args = dict(num_key_value_groups=groups, scaling=D ** -0.5, warm_format=odecode.WARM_ABSMAX_I8,
                cold_mode=odecode.COLD_MASKED if cold == "masked" else odecode.COLD_ZERO_LOGIT, return_scores=True)
    out, sc = odecode.decode_attention(q, table[None], states[None], lengths[None], nb, hk, hv, wk, wv, sk, None,
                                       sv, None, **args)
    ph, pw = rng.permutation(hk.shape[0]), rng.permutation(wk.shape[0])   # new slot of old slot i
    t2 = table.copy()
    t2[states == 0] = ph[table[states == 0]]
    t2[states == 1] = pw[table[states == 1]]
    hk2, hv2, wk2, wv2 = (np.empty_like(a) for a in (hk, hv, wk, wv))
    sk2, sv2 = np.empty_like(sk), np.empty_like(sv)
    hk2[ph], hv2[ph] = hk, hv
    wk2[pw], wv2[pw], sk2[pw], sv2[pw] = wk, wv, sk, sv
    out2, sc2 = odecode.decode_attention(q, t2[None], states[None], lengths[None], nb, hk2, hv2, wk2, wv2, sk2, None,
                                         sv2, None, **args)
    np.testing.assert_array_equal(out, out2)
    np.testing.assert_array_equal(sc, sc2)


@settings(**SETTINGS)
@given(st.integers(0, 2 ** 31 - 1), st.integers(1, 12), st.sampled_from([1, 2, 4]))
def test_all_hot_decode_is_dense_softmax_attention(seed, nb, groups):
    rng = np.random.default_rng(seed)
    kv, D, bs = 2, 16, 16
    states, table, lengths, hk, hv, _, _, _, _ = _compact_case(rng, nb, nb, 0, kv, D)
    wk = np.zeros((1, kv, bs, D), np.int8)
    s1 = np.ones((1, kv), np.float32)
    q = rng.standard_normal((1, kv * groups, D)).astype(np.float16)
    out = odecode.decode_attention(q, table[None], states[None], lengths[None], nb, hk, hv, wk, wk, s1, None, s1,
                                   None, groups, D ** -0.5, warm_format=odecode.WARM_ABSMAX_I8,
                                   cold_mode=odecode.COLD_MASKED)
    ks = np.concatenate([hk[table[i], :, :lengths[i]] for i in range(nb)], axis=1).astype(np.float64)
    vs = np.concatenate([hv[table[i], :, :lengths[i]] for i in range(nb)], axis=1).astype(np.float64)
    for h in range(kv * groups):
        logits = ks[h // groups] @ q[0, h].astype(np.float64) * np.float64(np.float32(D ** -0.5))
        p = np.exp(logits - logits.max())
        p /= p.sum()
        np.testing.assert_allclose(out[0, h], p @ vs[h // groups], rtol=1e-12, atol=1e-12)


@settings(**SETTINGS)
@given(st.integers(0, 2 ** 31 - 1), st.integers(1, 40), st.integers(0, 45), st.integers(0, 45))
def test_label_counts_follow_the_budgets(seed, n, hot, warm):
    rng = np.random.default_rng(seed)
    scores = rng.standard_normal((1, n)).astype(np.float32)
    cur = np.zeros((1, n), np.int32)                      # no sticky COLD
    lab = policy.tier_labels(scores, cur, hot, warm, "hot_warm_cold")[0]
    if n <= 2:
        assert (lab == 0).all()
        return
    n_hot = 2 + min(max(hot - 2, 0), n - 2)
    n_warm = min(max(warm, 0), n - n_hot)
    assert (lab == 0).sum() == n_hot and (lab == 1).sum() == n_warm and (lab == 2).sum() == n - n_hot - n_warm
    assert lab[0] == 0 and lab[-1] == 0
    # The HOT candidates are the highest-scoring ones.
    cand = scores[0, 1:-1]
    hot_c = cand[lab[1:-1] == 0]
    rest = cand[lab[1:-1] != 0]
    if hot_c.size and rest.size:
        assert hot_c.min() >= rest.max()

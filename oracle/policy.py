"""Block scores and tier labels (oracle; test infrastructure only).

* ``compute_block_scores`` restates TierKVPolicyEngine.compute_block_scores
  (tierkv_policy.py:1380-1389): mean over (batch, head, query), then the mean
  of each block_size chunk.
* ``block_scores_from_probability_sums`` restates
  TieredKVRuntime.block_scores_from_probability_sums (tierkv_policy.py:1905-1912).
* ``enforce_budget`` / ``enforce_tiered_budget`` restate the policy engine
  (tierkv_policy.py:1391-1432, 1434-1477) as pure functions returning the
  desired per-block states: reserved HOT {0, n-1} (n <= 2 -> all HOT);
  candidates sorted by score descending with Python's stable ``sorted`` (ties
  keep ascending index order); top hot_budget-2 HOT, next warm_budget WARM,
  rest COLD (tiered) or ``demoted_state``; a COLD block never leaves COLD.
* ``desired_prefill_states`` restates TieredKVRuntime._desired_prefill_states
  (tierkv_policy.py:1695-1720).
* ``block_mass_from_probs`` / ``block_mass_from_sums`` define the HIP
  block-score kernels' fixed reduction order (BASELINE config 2(b)):
  per token a sequential fp32 sum over heads h = 0..H-1, then a pairwise
  tree over the block's tokens ((t0+t1)+(t2+t3))+..., then ``/ H`` and
  ``/ max(len, 1)`` (two IEEE fp32 divisions).  The reference's own mean is
  the same quantity; its exact fp32 bits depend on ATen's reduction order,
  which is parity unpinned (labels are compared bit-exactly given identical
  scores).
* ``tier_labels`` batches ``enforce_tiered_budget`` / ``enforce_budget`` over
  sequences with a rank-by-counting formulation (rank_i = #{j: s_j > s_i or
  (s_j == s_i and j < i)}) that equals the stable descending sort.
* ``prefill_block_mass`` is ``compute_block_scores`` applied per sequence to
  the causal prefill attention probabilities, in float64 (the quantity the
  prefill block-score kernel computes without materialising them); pinned by
  closed forms (zero keys give p = 1 / (q + 1); one token gives mass 1;
  length-weighted masses sum to 1; a dominant key takes its queries' mass).

Pinned by the reference's known answer (main.py:375-389: block means
[0.4, 0.9, 0.1, 0.2], hot_budget 3 -> [0, 0, 1, 0]), its mode checks
(main.py:705-719), and by Python's ``sorted`` on random and tied inputs.
"""

from __future__ import annotations

import numpy as np

from . import COLD_STATE, HOT_STATE, WARM_STATE


def compute_block_scores(attn_weights, block_size):
    """tierkv_policy.py:1380-1389."""
    a = np.asarray(attn_weights, dtype=np.float64)
    if a.ndim != 4:
        raise ValueError("attn_weights must have shape [batch, num_heads, query_seq_len, past_seq_len].")
    if a.shape[-1] == 0:
        raise ValueError("attn_weights past_seq_len must be positive.")
    reduced = a.mean(axis=(0, 1, 2))
    return np.array([chunk.mean() for chunk in np.split(reduced, range(block_size, len(reduced), block_size))])


def block_scores_from_probability_sums(score_sums, lengths, num_blocks):
    """tierkv_policy.py:1905-1912: mean over heads of the per-block sums,
    divided by max(length, 1)."""
    n = int(num_blocks)
    if n == 0:
        return np.zeros(0, np.float64)
    s = np.asarray(score_sums, dtype=np.float64)[:, :n].mean(axis=0)
    return s / np.maximum(np.asarray(lengths[:n], dtype=np.float64), 1.0)


def _rank_candidates(scores, candidates):
    return sorted(candidates, key=lambda idx: float(scores[idx]), reverse=True)


def enforce_budget(scores, current_states, hot_budget, demoted_state=WARM_STATE):
    """tierkv_policy.py:1391-1432; returns the full new state list."""
    n = len(current_states)
    cur = [int(s) for s in current_states]
    if n == 0:
        return []
    if demoted_state not in (WARM_STATE, COLD_STATE):
        raise ValueError("demoted_state must be WARM_STATE or COLD_STATE.")
    if len(scores) != n:
        raise ValueError("block_scores length must match the allocated block count.")
    if n <= 2:
        return [HOT_STATE] * n
    reserved = {0, n - 1}
    extra_hot = max(int(hot_budget) - len(reserved), 0)
    ranked = _rank_candidates(scores, [i for i in range(n) if i not in reserved])
    hot = set(ranked[:extra_hot])
    out = []
    for i in range(n):
        desired = HOT_STATE if (i in reserved or i in hot) else demoted_state
        if cur[i] == COLD_STATE and desired != COLD_STATE:
            desired = COLD_STATE
        out.append(desired)
    return out


def enforce_tiered_budget(scores, current_states, hot_budget, warm_budget):
    """tierkv_policy.py:1434-1477; returns the full new state list."""
    n = len(current_states)
    cur = [int(s) for s in current_states]
    if n == 0:
        return []
    if len(scores) != n:
        raise ValueError("block_scores length must match the allocated block count.")
    if n <= 2:
        return [HOT_STATE] * n
    reserved = {0, n - 1}
    ranked = _rank_candidates(scores, [i for i in range(n) if i not in reserved])
    extra_hot = max(int(hot_budget) - len(reserved), 0)
    hot = set(ranked[:extra_hot])
    warm = set(ranked[extra_hot: extra_hot + max(int(warm_budget), 0)])
    out = []
    for i in range(n):
        if i in reserved or i in hot:
            desired = HOT_STATE
        elif i in warm:
            desired = WARM_STATE
        else:
            desired = COLD_STATE
        if cur[i] == COLD_STATE and desired != COLD_STATE:
            desired = COLD_STATE
        out.append(desired)
    return out


def desired_prefill_states(num_blocks, scores, hot_budget, warm_budget, policy_mode, demoted_state=WARM_STATE):
    """tierkv_policy.py:1695-1720."""
    n = int(num_blocks)
    if policy_mode == "hot_only" or n <= 2:
        return [HOT_STATE] * n
    if len(scores) != n:
        raise ValueError("block_scores must be a 1D tensor matching prefill block count.")
    reserved = {0, n - 1}
    ranked = _rank_candidates(scores, [i for i in range(n) if i not in reserved])
    extra_hot = max(int(hot_budget) - len(reserved), 0)
    hot = set(ranked[:extra_hot])
    if policy_mode == "hot_warm_cold":
        warm = set(ranked[extra_hot: extra_hot + max(int(warm_budget), 0)])
        return [HOT_STATE if (i in reserved or i in hot) else (WARM_STATE if i in warm else COLD_STATE)
                for i in range(n)]
    return [HOT_STATE if (i in reserved or i in hot) else demoted_state for i in range(n)]


def block_mass_from_probs(probs, block_size, lengths=None):
    """Fixed-order per-block mass of probabilities [B, H, T] -> [B, T/bs] fp32.

    lengths: optional [B, nblk] valid-token counts (default: full blocks);
    tokens beyond a block's length are excluded."""
    p = np.asarray(probs, dtype=np.float32)
    batch, heads, tokens = p.shape
    assert tokens % block_size == 0 and (block_size & (block_size - 1)) == 0
    nblk = tokens // block_size
    if lengths is None:
        lengths = np.full((batch, nblk), block_size, np.int64)
    lengths = np.asarray(lengths)
    tok = np.zeros((batch, tokens), np.float32)
    for h in range(heads):                      # sequential over heads
        tok = (tok + p[:, h, :]).astype(np.float32)
    pos = np.arange(tokens) % block_size
    valid = pos[None, :] < np.repeat(lengths, block_size, axis=1)
    tok = np.where(valid, tok, np.float32(0))
    x = tok.reshape(batch, nblk, block_size)
    while x.shape[-1] > 1:                      # pairwise tree over tokens
        x = (x[..., 0::2] + x[..., 1::2]).astype(np.float32)
    s = x[..., 0]
    s = (s / np.float32(heads)).astype(np.float32)
    return (s / np.maximum(lengths, 1).astype(np.float32)).astype(np.float32)


def block_mass_from_sums(score_sums, lengths, num_blocks):
    """Fixed-order restatement of block_scores_from_probability_sums for
    batched sums [B, H, maxB]: sequential fp32 sum over heads, ``/ H``,
    ``/ max(len, 1)``.  Returns [B, n] fp32."""
    s = np.asarray(score_sums, dtype=np.float32)
    batch, heads, _ = s.shape
    n = int(num_blocks)
    acc = np.zeros((batch, n), np.float32)
    for h in range(heads):
        acc = (acc + s[:, h, :n]).astype(np.float32)
    acc = (acc / np.float32(heads)).astype(np.float32)
    return (acc / np.maximum(np.asarray(lengths)[:, :n], 1).astype(np.float32)).astype(np.float32)


def tier_labels(scores, current_states, hot_budget, warm_budget, mode="hot_warm_cold", demoted_state=WARM_STATE):
    """Batched labels [B, n] via the reference's per-sequence rules."""
    scores = np.asarray(scores)
    cur = np.asarray(current_states)
    out = np.empty(cur.shape, np.int32)
    for b in range(cur.shape[0]):
        if mode == "hot_warm_cold":
            out[b] = enforce_tiered_budget(list(scores[b]), list(cur[b]), hot_budget, warm_budget)
        elif mode == "hot_warm":
            out[b] = enforce_budget(list(scores[b]), list(cur[b]), hot_budget, demoted_state)
        elif mode == "hot_only":
            out[b] = cur[b]  # enforce_policy returns early (tierkv_policy.py:1888-1889)
        else:
            raise ValueError(mode)
    return out


def prefill_block_mass(q, k, scaling, block_size):
    """Per-sequence prefill block scores: compute_block_scores
    (tierkv_policy.py:1380-1389) applied to one sequence's causal attention
    probabilities (eager_attention_forward, modeling_llama.py:225-247: fp32
    softmax of scaling * q . k with the causal mask), here in float64 without
    the reference's fp16 rounding of the probabilities.

    q [B, H, T, D], k [B, H_kv, T, D] -> [B, ceil(T / block_size)]: the mean
    probability over heads and queries, averaged over each block's tokens.
    Materialises [H, T, T] per sequence: small T only."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    B, H, T, _ = q.shape
    G = H // k.shape[1]
    nblk = -(-T // block_size)
    out = np.zeros((B, nblk))
    causal = np.tril(np.ones((T, T), bool))
    for b in range(B):
        kk = np.repeat(k[b], G, axis=0)                       # [H, T, D]
        logits = np.einsum("hqd,htd->hqt", q[b], kk) * scaling
        logits = np.where(causal[None], logits, -np.inf)
        logits -= logits.max(axis=-1, keepdims=True)
        p = np.exp(logits)
        p /= p.sum(axis=-1, keepdims=True)
        per_token = p.sum(axis=(0, 1)) / (H * T)              # mean over heads and queries
        for blk in range(nblk):
            out[b, blk] = per_token[blk * block_size:(blk + 1) * block_size].mean()
    return out

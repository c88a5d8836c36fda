"""Tiered paged decode attention (oracle; test infrastructure only).

Restates ``_eager_reference_decode`` (tierkv_triton.py:708-820) and the
kernel's optional score pass (tierkv_triton.py:121-145), generalised to a
batch of sequences (one table row per sequence) and to the two warm formats
and two COLD semantics the HIP path supports:

* HOT block: fp16 K/V read from ``hot_k/hot_v[slot]`` (tierkv_triton.py:92-93,
  770-773).
* WARM block, reference format: ``(u8 - zero) * scale`` in fp32 with fp16
  per-token scale/zero (tierkv_triton.py:95-102, 757-767).
  WARM block, absmax format: ``int8 * scale`` with an fp32 scale per
  (slot, kv head).
* COLD block, ``zero_logit`` (reference): K = V = 0 for the block's valid
  tokens, which still enter the softmax with logit 0
  (tierkv_triton.py:92-102 masked loads -> 0; eager 768-774).
  COLD block, ``masked``: the block contributes no tokens (
  "cold evicted (masked out)").
* Tokens ``t >= block_lengths[b]`` are invalid (tierkv_triton.py:104-106, 777).
* GQA: q head ``h`` reads kv head ``h // groups`` (tierkv_triton.py:71, 790-792).
* Softmax in float64 over all valid tokens; an all-invalid row gives 0
  (``nan_to_num``, tierkv_triton.py:804-805).
* Score pass: per (q head, logical block) ``sum_{valid t in block} p_t``
  (tierkv_triton.py:121-145); zero beyond ``num_blocks``.

Pinned by: textbook softmax attention on all-HOT inputs (tests compare with
an independent dense implementation and torch SDPA), closed-form COLD
identities (all-COLD zero_logit -> exactly 0; masked COLD == zero-length
block), GQA with groups=1 == per-head MHA, and the reference's score
normalisation (sum over blocks == 1, tierkv_triton.py:933-937).
"""

from __future__ import annotations

import numpy as np

from . import COLD_STATE, HOT_STATE, WARM_STATE

WARM_REF_U8 = "ref_u8"
WARM_ABSMAX_I8 = "absmax_i8"
COLD_ZERO_LOGIT = "zero_logit"
COLD_MASKED = "masked"


def gather_sequence_kv(
    table_row, states_row, lengths_row, num_blocks,
    hot_k, hot_v, warm_k, warm_v, k_scale, k_zero, v_scale, v_zero,
    warm_format, cold_mode,
):
    """Per-block gather/dequant of one sequence (tierkv_triton.py:747-781).

    Returns (K [H_kv, T, D] f32, V [H_kv, T, D] f32, valid [T] bool,
    block_of_token [T] int) for the tokens that enter the softmax.
    """
    kv_heads, block_size, head_dim = hot_k.shape[1], hot_k.shape[2], hot_k.shape[3]
    ks, vs, valids, owners = [], [], [], []
    for b in range(int(num_blocks)):
        slot = int(table_row[b])
        state = int(states_row[b])
        blen = int(lengths_row[b])
        valid = np.arange(block_size) < blen
        if state == HOT_STATE:
            kb = hot_k[slot].astype(np.float32)
            vb = hot_v[slot].astype(np.float32)
        elif state == WARM_STATE:
            if warm_format == WARM_REF_U8:
                kb = (warm_k[slot].astype(np.float32) - k_zero[slot].astype(np.float32)) * k_scale[slot].astype(np.float32)
                vb = (warm_v[slot].astype(np.float32) - v_zero[slot].astype(np.float32)) * v_scale[slot].astype(np.float32)
            elif warm_format == WARM_ABSMAX_I8:
                kb = warm_k[slot].astype(np.float32) * k_scale[slot].astype(np.float32)[:, None, None]
                vb = warm_v[slot].astype(np.float32) * v_scale[slot].astype(np.float32)[:, None, None]
            else:
                raise ValueError(f"unknown warm format {warm_format!r}")
        elif state == COLD_STATE:
            kb = np.zeros((kv_heads, block_size, head_dim), np.float32)
            vb = np.zeros((kv_heads, block_size, head_dim), np.float32)
            if cold_mode == COLD_MASKED:
                valid = np.zeros(block_size, dtype=bool)
            elif cold_mode != COLD_ZERO_LOGIT:
                raise ValueError(f"unknown cold mode {cold_mode!r}")
        else:
            raise ValueError(f"unsupported block state {state}")
        ks.append(kb)
        vs.append(vb)
        valids.append(valid)
        owners.append(np.full(block_size, b, dtype=np.int64))
    return (np.concatenate(ks, axis=1), np.concatenate(vs, axis=1),
            np.concatenate(valids), np.concatenate(owners))


def decode_attention(
    query, block_table, block_states, block_lengths, num_blocks,
    hot_k, hot_v, warm_k, warm_v, k_scale, k_zero, v_scale, v_zero,
    num_key_value_groups, scaling,
    warm_format=WARM_REF_U8, cold_mode=COLD_ZERO_LOGIT, return_scores=False,
):
    """Batched oracle decode.

    query: [B, H, D] (any float dtype).  block_table/states/lengths:
    [B, maxB] int.  num_blocks: int or [B] ints.  Returns out [B, H, D]
    float64 and, if ``return_scores``, score_sums [B, H, maxB] float64.
    """
    query = np.asarray(query)
    batch, num_heads, head_dim = query.shape
    max_blocks = np.asarray(block_table).shape[1]
    nb = np.broadcast_to(np.asarray(num_blocks, dtype=np.int64), (batch,))
    out = np.zeros((batch, num_heads, head_dim), np.float64)
    scores = np.zeros((batch, num_heads, max_blocks), np.float64)
    groups = int(num_key_value_groups)
    for bi in range(batch):
        k, v, valid, owner = gather_sequence_kv(
            block_table[bi], block_states[bi], block_lengths[bi], nb[bi],
            hot_k, hot_v, warm_k, warm_v, k_scale, k_zero, v_scale, v_zero,
            warm_format, cold_mode)
        # GQA expansion (repeat_interleave, tierkv_triton.py:790-792).
        k_exp = np.repeat(k, groups, axis=0).astype(np.float64)
        v_exp = np.repeat(v, groups, axis=0).astype(np.float64)
        q = query[bi].astype(np.float32).astype(np.float64)
        logits = np.einsum("hd,htd->ht", q, k_exp) * float(np.float32(scaling))
        logits = np.where(valid[None, :], logits, -np.inf)
        if not valid.any():
            continue  # softmax of an all -inf row -> nan -> 0
        m = logits.max(axis=-1, keepdims=True)
        e = np.where(valid[None, :], np.exp(logits - m), 0.0)
        p = e / e.sum(axis=-1, keepdims=True)
        out[bi] = np.einsum("ht,htd->hd", p, v_exp)
        if return_scores:
            np.add.at(scores[bi].T, owner, p.T)
    if return_scores:
        return out, scores
    return out


def ideal_bytes(states, num_blocks, num_heads, num_kv_heads, head_dim, block_size=16,
                warm_format=WARM_ABSMAX_I8, return_scores=False):
    """Algorithmic HBM bytes of one decode launch.

    Per sequence: HOT blocks 2*H_kv*bs*D*2 (K+V fp16); WARM blocks
    2*H_kv*bs*D*1 plus metadata (absmax: 2*H_kv*4; reference format:
    2*2*H_kv*bs*2 per-token fp16 scale+zero); COLD 0; 12 B of table, state and
    length per block; q in and out 2*H*D*2.  Score output adds H*n_blocks*4.
    """
    states = np.asarray(states)
    nb = np.broadcast_to(np.asarray(num_blocks, dtype=np.int64), (states.shape[0],))
    if warm_format == WARM_ABSMAX_I8:
        warm_meta = 2 * num_kv_heads * 4
    else:
        warm_meta = 2 * 2 * num_kv_heads * block_size * 2
    total = 0
    for bi in range(states.shape[0]):
        row = states[bi, : nb[bi]]
        n_hot = int((row == HOT_STATE).sum())
        n_warm = int((row == WARM_STATE).sum())
        total += n_hot * 2 * num_kv_heads * block_size * head_dim * 2
        total += n_warm * (2 * num_kv_heads * block_size * head_dim + warm_meta)
        total += int(nb[bi]) * 12 + 2 * num_heads * head_dim * 2
        if return_scores:
            total += num_heads * int(nb[bi]) * 4
    return total

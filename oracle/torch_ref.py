"""The reference's CPU PyTorch decode path, restated in torch on the CPU
(test and baseline infrastructure only: ``bench.py``'s ``cpu_baseline`` leg
times it, ``tests/test_oracle_torch_ref.py`` checks it against
``oracle.decode``).

``eager_decode_looped`` keeps the structure of ``_eager_reference_decode``
(tierkv_triton.py:708-820), the reference's own CPU-runnable decode:

* a Python loop over the logical blocks that reads each block's slot, state
  and length with ``.item()`` (tierkv_triton.py:747-750);
* per block, the fp32 K/V of its tier: HOT read as is, WARM dequantized
  (the reference's ``(u8 - zero) * scale``, tierkv_triton.py:757-767, or the
  absmax ``i8 * scale``), COLD zeros (768-774), plus a ``[block_size]`` valid
  mask ``arange < length`` (777);
* ``torch.cat`` of the per-block K/V and masks (784-788), ``repeat_interleave``
  over the GQA group (790-792), fp32 logits, ``masked_fill(-inf)``, fp32
  ``softmax`` and ``nan_to_num`` (794-805), the value sum (808);
* a batch is served as a loop over sequences, one batch-1 call each, as the
  reference serves concurrent requests (main.py:1182-1189).

In the ``masked`` COLD mode (BASELINE's "evicted, masked out") a COLD block's
tokens are invalid instead of zero-logit.

``vectorized_decode`` computes the same quantity for the whole batch with
gathers and batched matrix products (no per-block Python): the stronger
torch-CPU number reported beside the looped one.
"""

from __future__ import annotations

import torch

from . import COLD_STATE, HOT_STATE, WARM_STATE


def _warm_block(warm_k, warm_v, k_scale, k_zero, v_scale, v_zero, slot, warm_format):
    if warm_format == "ref_u8":
        k = (warm_k[slot].float() - k_zero[slot].float()) * k_scale[slot].float()
        v = (warm_v[slot].float() - v_zero[slot].float()) * v_scale[slot].float()
    else:
        k = warm_k[slot].float() * k_scale[slot].float()[:, None, None]
        v = warm_v[slot].float() * v_scale[slot].float()[:, None, None]
    return k, v


def eager_decode_one(query, table, states, lengths, hot_k, hot_v, warm_k, warm_v, k_scale, k_zero, v_scale,
                     v_zero, num_blocks, groups, scaling, warm_format="ref_u8", cold_mode="zero_logit"):
    """One sequence: query [1, H, 1, D]; table/states/lengths 1-D int32.
    Returns [1, 1, H, D] in the query dtype (tierkv_triton.py:708-820)."""
    block_size = hot_k.shape[2]
    ks, vs, valids = [], [], []
    for blk in range(int(num_blocks)):
        slot = max(int(table[blk].item()), 0)
        state = int(states[blk].item())
        length = int(lengths[blk].item())
        valid = torch.arange(block_size) < length
        if state == WARM_STATE:
            k, v = _warm_block(warm_k, warm_v, k_scale, k_zero, v_scale, v_zero, slot, warm_format)
        elif state == HOT_STATE:
            k, v = hot_k[slot].float(), hot_v[slot].float()
        else:
            k = torch.zeros(hot_k.shape[1:], dtype=torch.float32)
            v = torch.zeros_like(k)
            if state == COLD_STATE and cold_mode == "masked":
                valid = torch.zeros(block_size, dtype=torch.bool)
        ks.append(k)
        vs.append(v)
        valids.append(valid)
    k_all = torch.cat(ks, dim=1).repeat_interleave(groups, dim=0)
    v_all = torch.cat(vs, dim=1).repeat_interleave(groups, dim=0)
    valid_all = torch.cat(valids)
    q = query[0, :, 0, :].float()
    logits = torch.einsum("hd,htd->ht", q, k_all) * scaling
    logits = logits.masked_fill(~valid_all.unsqueeze(0), float("-inf"))
    probs = torch.nan_to_num(torch.softmax(logits, dim=-1), nan=0.0)
    out = torch.einsum("ht,htd->hd", probs, v_all)
    return out.view(1, 1, *out.shape).to(query.dtype)


def eager_decode_looped(query, table, states, lengths, hot_k, hot_v, warm_k, warm_v, k_scale, k_zero, v_scale,
                        v_zero, num_blocks, groups, scaling, warm_format="ref_u8", cold_mode="zero_logit"):
    """A batch as a loop over sequences: query [B, H, 1, D], tables [B, maxB]
    -> [B, 1, H, D]."""
    outs = []
    for b in range(query.shape[0]):
        outs.append(eager_decode_one(query[b:b + 1], table[b], states[b], lengths[b], hot_k, hot_v, warm_k,
                                     warm_v, k_scale, k_zero, v_scale, v_zero, num_blocks, groups, scaling,
                                     warm_format, cold_mode))
    return torch.cat(outs, dim=0)


def vectorized_decode(query, table, states, lengths, hot_k, hot_v, warm_k, warm_v, k_scale, k_zero, v_scale,
                      v_zero, num_blocks, groups, scaling, warm_format="ref_u8", cold_mode="zero_logit"):
    """The same decode for the whole batch with gathers and batched products:
    query [B, H, 1, D], tables [B, maxB] -> [B, 1, H, D]."""
    n = int(num_blocks)
    B, H, _, D = query.shape
    kv, bs = hot_k.shape[1], hot_k.shape[2]
    slot = table[:, :n].long().clamp(min=0)
    st = states[:, :n]
    hot_sel = (st == HOT_STATE).view(B, n, 1, 1, 1)
    warm_sel = (st == WARM_STATE).view(B, n, 1, 1, 1)
    hs = slot.clamp(max=hot_k.shape[0] - 1)
    ws = slot.clamp(max=warm_k.shape[0] - 1)
    k = torch.where(hot_sel, hot_k[hs].float(), 0.0)
    v = torch.where(hot_sel, hot_v[hs].float(), 0.0)
    if warm_format == "ref_u8":
        wk = (warm_k[ws].float() - k_zero[ws].float()) * k_scale[ws].float()
        wv = (warm_v[ws].float() - v_zero[ws].float()) * v_scale[ws].float()
    else:
        wk = warm_k[ws].float() * k_scale[ws].float()[..., None, None]
        wv = warm_v[ws].float() * v_scale[ws].float()[..., None, None]
    k = torch.where(warm_sel, wk, k)                       # [B, n, kv, bs, D]
    v = torch.where(warm_sel, wv, v)
    valid = torch.arange(bs).view(1, 1, bs) < lengths[:, :n].view(B, n, 1)
    if cold_mode == "masked":
        valid = valid & (st != COLD_STATE).view(B, n, 1)
    k = k.permute(0, 2, 1, 3, 4).reshape(B, kv, n * bs, D)
    v = v.permute(0, 2, 1, 3, 4).reshape(B, kv, n * bs, D)
    q = query[:, :, 0, :].float().view(B, kv, groups, D)
    logits = torch.matmul(q, k.transpose(2, 3)) * scaling          # [B, kv, G, T]
    logits = logits.masked_fill(~valid.view(B, 1, 1, n * bs), float("-inf"))
    probs = torch.nan_to_num(torch.softmax(logits, dim=-1), nan=0.0)
    out = torch.matmul(probs, v).reshape(B, H, D)
    return out.view(B, 1, H, D).to(query.dtype)

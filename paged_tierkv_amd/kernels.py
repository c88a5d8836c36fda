"""Python entry points of the demotion, promotion, block-score and label
kernels (C ABI in include/tierkv_hip.h).

All tensors are GPU tensors; index arrays are int32.  Launches are
asynchronous on the current stream.
"""

from __future__ import annotations

import torch

from . import _lib

WARM_FORMATS = {"ref_u8": _lib.WARM_REF_U8, "absmax_i8": _lib.WARM_ABSMAX_I8}
LABEL_MODES = {"hot_only": 0, "hot_warm": 1, "hot_warm_cold": 2}


def _i32(x, device) -> torch.Tensor:
    t = torch.as_tensor(x, dtype=torch.int32)
    return t.to(device).contiguous()


def _table_positions(table_pos, block_table, block_states, n, device):
    """Validate (on the host, where the positions usually come from) and
    upload the flat table positions of a migration batch."""
    if table_pos is None:
        return None
    if block_table is None or block_states is None:
        raise ValueError("table_pos needs block_table and block_states.")
    host = torch.as_tensor(table_pos, dtype=torch.int32)
    if host.numel() != n:
        raise ValueError("table_pos needs one entry per job.")
    if host.device.type == "cpu" and host.numel():
        hi = int(host.max())
        if hi >= min(block_table.numel(), block_states.numel()):
            raise ValueError("table_pos entry outside the block table.")
    return host.to(device).contiguous()


def _check_tiles(t: torch.Tensor, name: str, dtype) -> None:
    _lib.require_gpu_tensor(t, name)
    if t.dtype != dtype or t.ndim != 4 or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous {dtype} [tiles, kv_heads, block_size, head_dim] tensor.")


def demote_to_warm(src_k, src_v, src_index, dst_slot, lengths, warm_k, warm_v, k_scale, k_zero,
                   v_scale, v_zero, warm_format: str = "ref_u8", pad_tail: bool = False,
                   block_table=None, block_states=None, table_pos=None):
    """Quantize fp16 tiles ``src_k/src_v[src_index[i]]`` (first ``lengths[i]``
    tokens) into WARM slots ``dst_slot[i]``; optionally rewrite
    ``block_table/block_states`` at flat positions ``table_pos`` to
    (dst_slot, WARM).  Batched CompactTieredKVTensorPool.demote_to_warm
    (tierkv_policy.py:1042-1068) / write_warm_block (969-1002)."""
    lib = _lib.lib()
    fmt = WARM_FORMATS[warm_format]
    _check_tiles(src_k, "src_k", torch.float16)
    _check_tiles(src_v, "src_v", torch.float16)
    _check_tiles(warm_k, "warm_k", torch.uint8 if fmt == _lib.WARM_REF_U8 else torch.int8)
    _check_tiles(warm_v, "warm_v", warm_k.dtype)
    kv_heads, bs, dim = (int(x) for x in src_k.shape[1:])
    if tuple(warm_k.shape[1:]) != (kv_heads, bs, dim) or src_v.shape != src_k.shape or warm_v.shape != warm_k.shape:
        raise ValueError("source and WARM pool geometry differ.")
    device = src_k.device
    src_index = _i32(src_index, device)
    dst_slot = _i32(dst_slot, device)
    lengths = _i32(lengths, device)
    n = int(src_index.numel())
    if dst_slot.numel() != n or lengths.numel() != n:
        raise ValueError("src_index, dst_slot and lengths must have the same length.")
    tp = _table_positions(table_pos, block_table, block_states, n, device)
    rc = lib.tierkv_demote_to_warm(
        _lib.ptr(src_k), _lib.ptr(src_v), int(src_k.shape[0]),
        _lib.ptr(src_index), _lib.ptr(dst_slot), _lib.ptr(lengths), n,
        _lib.ptr(warm_k), _lib.ptr(warm_v), int(warm_k.shape[0]),
        _lib.ptr(k_scale), _lib.ptr(k_zero), _lib.ptr(v_scale), _lib.ptr(v_zero),
        fmt, int(bool(pad_tail)),
        _lib.ptr(block_table), _lib.ptr(block_states), _lib.ptr(tp),
        kv_heads, bs, dim, _lib.stream_of(device))
    _lib.check(rc, "tierkv_demote_to_warm")


def promote_to_hot(warm_k, warm_v, k_scale, k_zero, v_scale, v_zero, src_slot, dst_slot, lengths,
                   hot_k, hot_v, warm_format: str = "ref_u8",
                   block_table=None, block_states=None, table_pos=None):
    """Dequantize WARM slots into HOT slots (promote_to_hot,
    tierkv_policy.py:1087-1115, with dequantize_int8_to_fp16, 39-44)."""
    lib = _lib.lib()
    fmt = WARM_FORMATS[warm_format]
    _check_tiles(hot_k, "hot_k", torch.float16)
    _check_tiles(hot_v, "hot_v", torch.float16)
    _check_tiles(warm_k, "warm_k", torch.uint8 if fmt == _lib.WARM_REF_U8 else torch.int8)
    kv_heads, bs, dim = (int(x) for x in hot_k.shape[1:])
    device = hot_k.device
    src_slot = _i32(src_slot, device)
    dst_slot = _i32(dst_slot, device)
    lengths = _i32(lengths, device)
    n = int(src_slot.numel())
    tp = _table_positions(table_pos, block_table, block_states, n, device)
    rc = lib.tierkv_promote_to_hot(
        _lib.ptr(warm_k), _lib.ptr(warm_v), int(warm_k.shape[0]),
        _lib.ptr(k_scale), _lib.ptr(k_zero), _lib.ptr(v_scale), _lib.ptr(v_zero),
        _lib.ptr(src_slot), _lib.ptr(dst_slot), _lib.ptr(lengths), n,
        _lib.ptr(hot_k), _lib.ptr(hot_v), int(hot_k.shape[0]), fmt,
        _lib.ptr(block_table), _lib.ptr(block_states), _lib.ptr(tp),
        kv_heads, bs, dim, _lib.stream_of(device))
    _lib.check(rc, "tierkv_promote_to_hot")


def block_mass_from_probs(probs: torch.Tensor, block_size: int, lengths: torch.Tensor | None = None,
                          out: torch.Tensor | None = None):
    """fp32 probabilities [B, H, T] -> per-block mass [B, T / block_size]
    (written into ``out`` when given: contiguous fp32 of that shape)."""
    lib = _lib.lib()
    _lib.require_gpu_tensor(probs, "probs")
    if probs.dtype != torch.float32 or probs.ndim != 3:
        raise ValueError("probs must be fp32 [batch, heads, tokens].")
    probs = probs.contiguous()
    batch, heads, tokens = (int(x) for x in probs.shape)
    if tokens % int(block_size):
        raise ValueError("tokens must be a multiple of block_size.")
    nblk = tokens // int(block_size)
    if out is None:
        out = torch.empty((batch, nblk), dtype=torch.float32, device=probs.device)
    elif (out.dtype != torch.float32 or tuple(out.shape) != (batch, nblk) or not out.is_contiguous()
          or out.device != probs.device):
        raise ValueError("out must be a contiguous fp32 [batch, tokens / block_size] tensor on the probs' device.")
    if lengths is not None:
        lengths = _i32(lengths, probs.device)
        if tuple(lengths.shape) != (batch, nblk):
            raise ValueError("lengths must be [batch, tokens / block_size].")
    rc = lib.tierkv_block_mass_from_probs(_lib.ptr(probs), _lib.ptr(lengths), _lib.ptr(out),
                                          batch, heads, tokens, int(block_size), _lib.stream_of(probs.device))
    _lib.check(rc, "tierkv_block_mass_from_probs")
    return out


def block_scores_from_sums(score_sums: torch.Tensor, lengths: torch.Tensor, num_blocks: int):
    """block_scores_from_probability_sums (tierkv_policy.py:1905-1912):
    score_sums [H, maxB] / [B, H, maxB], lengths [maxB] / [B, maxB] ->
    [n] / [B, n] fp32."""
    lib = _lib.lib()
    squeeze = score_sums.ndim == 2
    s = score_sums.unsqueeze(0) if squeeze else score_sums
    ln = lengths.unsqueeze(0) if lengths.ndim == 1 else lengths
    s = s.contiguous()
    ln = ln.to(torch.int32).contiguous()
    batch, heads, stride = (int(x) for x in s.shape)
    n = int(num_blocks)
    out = torch.empty((batch, n), dtype=torch.float32, device=s.device)
    rc = lib.tierkv_block_scores_from_sums(_lib.ptr(s), stride, _lib.ptr(ln), int(ln.shape[-1]), _lib.ptr(out),
                                           batch, heads, n, _lib.stream_of(s.device))
    _lib.check(rc, "tierkv_block_scores_from_sums")
    return out[0] if squeeze else out


def tier_labels(scores: torch.Tensor, cur_states: torch.Tensor, hot_budget: int, warm_budget: int = 0,
                mode: str = "hot_warm_cold", demoted_state: int = 1, out: torch.Tensor | None = None):
    """enforce_tiered_budget / enforce_budget for a batch of sequences.
    scores fp32 [B, n] (or [n]); cur_states int32 [B, >= n] -> new states
    int32 of cur_states' shape (entries >= n copied unchanged)."""
    lib = _lib.lib()
    squeeze = scores.ndim == 1
    sc = (scores.unsqueeze(0) if squeeze else scores).to(torch.float32).contiguous()
    cur = (cur_states.unsqueeze(0) if cur_states.ndim == 1 else cur_states).to(torch.int32).contiguous()
    batch, n = (int(x) for x in sc.shape)
    if out is None:
        out = cur.clone()
    else:
        out = out.unsqueeze(0) if out.ndim == 1 else out
    rc = lib.tierkv_tier_labels(_lib.ptr(sc), _lib.ptr(cur), _lib.ptr(out), int(cur.shape[-1]), batch, n,
                                int(hot_budget), int(warm_budget), LABEL_MODES[mode], int(demoted_state),
                                _lib.stream_of(sc.device))
    _lib.check(rc, "tierkv_tier_labels")
    return out[0] if squeeze else out


_prefill_ws: dict = {}


def prefill_block_mass(query_states: torch.Tensor, key_states: torch.Tensor, block_size: int, scaling: float):
    """Per-sequence prefill block scores without materialised probabilities
    (``tierkv_prefill_block_mass``): query [B, H, T, D] and key [B, H_kv, T, D]
    (fp16 / bf16, any layout with head_dim contiguous, e.g. HF's transposed
    projections) -> fp32 [B, ceil(T / block_size)], the mean causal attention
    probability of each block over heads and queries (compute_block_scores,
    tierkv_policy.py:1380-1389, per sequence)."""
    lib = _lib.lib()
    _lib.require_gpu_tensor(query_states, "query_states")
    _lib.require_gpu_tensor(key_states, "key_states")
    if query_states.ndim != 4 or key_states.ndim != 4:
        raise ValueError("query and key states must be [batch, heads, tokens, head_dim].")
    if query_states.dtype not in (torch.float16, torch.bfloat16) or key_states.dtype != query_states.dtype:
        raise ValueError("query and key states must share an fp16 / bf16 dtype.")
    q, k = query_states, key_states
    if q.stride(-1) != 1 or q.stride(0) % 8 or q.stride(1) % 8 or q.stride(2) % 8 or q.data_ptr() % 16:
        q = q.contiguous()
    if k.stride(-1) != 1 or k.stride(0) % 8 or k.stride(1) % 8 or k.stride(2) % 8 or k.data_ptr() % 16:
        k = k.contiguous()
    batch, heads, tokens, dim = (int(x) for x in q.shape)
    if k.shape[0] != batch or k.shape[2] != tokens or k.shape[3] != dim:
        raise ValueError("key states do not match the query geometry.")
    kv_heads = int(k.shape[1])
    need = int(lib.tierkv_prefill_block_mass_workspace_bytes(batch, kv_heads, tokens))
    # One scratch buffer per (device, stream): launches on one stream are
    # ordered; launches on different streams may overlap and never share it.
    key = (q.device.index, _lib.stream_of(q.device))
    ws = _prefill_ws.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.empty(max(need, 256), dtype=torch.uint8, device=q.device)
        _prefill_ws[key] = ws
    nblk = (tokens + int(block_size) - 1) // int(block_size)
    out = torch.empty((batch, nblk), dtype=torch.float32, device=q.device)
    rc = lib.tierkv_prefill_block_mass(
        _lib.ptr(q), q.stride(0), q.stride(1), q.stride(2), _lib.ptr(k), k.stride(0), k.stride(1), k.stride(2),
        _lib.DTYPE_BF16 if q.dtype == torch.bfloat16 else _lib.DTYPE_F16, _lib.ptr(out), batch, heads, kv_heads,
        tokens, dim, int(block_size), float(scaling), _lib.ptr(ws), int(ws.numel()), _lib.stream_of(q.device))
    _lib.check(rc, "tierkv_prefill_block_mass")
    return out

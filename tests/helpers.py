"""Shared test helpers: quantize a workload's WARM sources with the oracle,
run the oracle decode, and move a case to the GPU."""

from __future__ import annotations

import numpy as np
import torch

from oracle import codec
from oracle import decode as odecode

ATOL = 2e-3   # BASELINE.json north_star tolerance vs the fp32 reference
RTOL = 1e-2


def oracle_warm(case, warm_format):
    """Quantize case.warm_src_* on the CPU with the oracle codec.
    Returns numpy (warm_k, warm_v, k_scale, k_zero, v_scale, v_zero)."""
    wk = case.warm_src_k.numpy()
    wv = case.warm_src_v.numpy()
    if warm_format == "absmax_i8":
        qk, sk = codec.quantize_absmax_i8(wk)
        qv, sv = codec.quantize_absmax_i8(wv)
        return qk, qv, sk, None, sv, None
    qk, sk, zk = codec.quantize_ref_u8(wk)
    qv, sv, zv = codec.quantize_ref_u8(wv)
    return qk, qv, sk, zk, sv, zv


def oracle_decode(case, warm, warm_format, cold_mode=None, return_scores=False, seqs=None):
    qk, qv, sk, zk, sv, zv = warm
    seqs = list(range(case.batch)) if seqs is None else list(seqs)
    q = case.query[seqs, :, 0, :].numpy()
    res = odecode.decode_attention(
        q, case.block_table[seqs].numpy(), case.block_states[seqs].numpy(), case.block_lengths[seqs].numpy(),
        case.num_blocks, case.hot_k.numpy(), case.hot_v.numpy(), qk, qv, sk, zk, sv, zv,
        case.groups, case.scaling, warm_format=warm_format, cold_mode=cold_mode or case.cold_mode,
        return_scores=return_scores)
    return res


def to_gpu_inputs(case, warm, device, query_dtype=torch.float16):
    qk, qv, sk, zk, sv, zv = warm
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(device)
    return dict(
        query_states=case.query.to(query_dtype).to(device),
        block_table=case.block_table.to(device), block_states=case.block_states.to(device),
        block_lengths=case.block_lengths.to(device),
        hot_k_pool=case.hot_k.to(device), hot_v_pool=case.hot_v.to(device),
        warm_k_pool=t(qk), warm_v_pool=t(qv), k_scale=t(sk), k_zero=t(zk), v_scale=t(sv), v_zero=t(zv),
        num_blocks=case.num_blocks, num_key_value_groups=case.groups, scaling=case.scaling)


def error_stats(actual, expected, atol=ATOL, rtol=RTOL) -> dict:
    """max |a - e|, max |a - e| / |e| over |e| >= atol, and the largest
    fraction of the tolerance atol + rtol |e| any element uses (< 1 passes)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    err = np.abs(a - e)
    big = np.abs(e) >= atol
    return {"max_abs": float(err.max()) if err.size else 0.0,
            "max_rel": float((err[big] / np.abs(e[big])).max()) if big.any() else 0.0,
            "tol_used": float((err / (atol + rtol * np.abs(e))).max()) if err.size else 0.0}


def assert_close(actual, expected, atol=ATOL, rtol=RTOL, what="output"):
    """Elementwise |a - e| <= atol + rtol |e|; returns error_stats."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, f"{what}: shape {a.shape} != {e.shape}"
    bad = ~(np.abs(a - e) <= atol + rtol * np.abs(e))
    if bad.any():
        idx = np.argwhere(bad)[:5].tolist()
        raise AssertionError(f"{what}: {int(bad.sum())} of {a.size} outside atol={atol} rtol={rtol}; "
                             f"max abs err {np.abs(a - e).max():.3e}; first bad {idx}")
    return error_stats(a, e, atol, rtol)


def report(what: str, stats: dict) -> None:
    print(f"[parity] {what}: max_abs={stats['max_abs']:.3e} max_rel={stats['max_rel']:.3e} "
          f"tol_used={stats['tol_used']:.3f} (atol {ATOL}, rtol {RTOL})", flush=True)

"""ctypes binding of ``libtierkv_hip.so`` (C ABI in include/tierkv_hip.h).

The library is loaded lazily and only from this package directory.  torch
is imported first so the process uses torch's HIP runtime (same soname).  A
missing library raises RuntimeError: there is no fallback path.
"""

from __future__ import annotations

import ctypes
import os
import threading
from ctypes import POINTER, c_char_p, c_float, c_int32, c_int64, c_void_p
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library links against)

LIB_PATH = Path(__file__).resolve().with_name("libtierkv_hip.so")
ABI_VERSION = 1

TIERKV_OK = 0
TIERKV_ERR_INVALID = 1
TIERKV_ERR_UNSUPPORTED = 2
TIERKV_ERR_HIP = 3
TIERKV_ERR_WORKSPACE = 4
TIERKV_ERR_STATE = 5

DTYPE_F16 = 0
DTYPE_BF16 = 1
WARM_REF_U8 = 0
WARM_ABSMAX_I8 = 1
COLD_ZERO_LOGIT = 0
COLD_MASKED = 1
DECODE_DETERMINISTIC = 0x40000000   # OR'ed into a decode call's splits hint

_P = c_void_p
_I32P = POINTER(c_int32)


class DecodeStep(ctypes.Structure):
    """TierkvDecodeStep (include/tierkv_hip.h): the token write, the table
    writes and the decode launch of one layer step, for tierkv_decode_step.
    The library's sizeof is checked against this layout when it loads."""

    _fields_ = [(name, _P) for name in (
        "src_k", "src_v", "hot_k", "hot_v", "table_dst", "query", "out", "score_sums", "block_table",
        "block_states", "block_lengths", "seq_num_blocks", "warm_k", "warm_v", "k_scale", "k_zero", "v_scale",
        "v_zero", "workspace")] + [(name, c_int64) for name in (
            "src_seqs", "hot_slots", "table_len", "table_stride", "warm_slots", "workspace_bytes")] + [
        (name, c_int32) for name in (
            "src_tokens", "n_jobs", "zero_tail", "n_pairs", "query_dtype", "num_blocks", "warm_format", "cold_mode",
            "batch", "num_heads", "num_kv_heads", "block_size", "head_dim")] + [
        ("scaling", c_float), ("splits_hint", c_int32), ("jobs", (c_int32 * 5) * 4), ("pairs", (c_int32 * 2) * 16)]

# name -> (restype, argtypes)
SIGNATURES = {
    "tierkv_last_error": (c_char_p, []),
    "tierkv_abi_version": (c_int32, []),
    "tierkv_decode_attention": (c_int32, [
        _P, c_int32, _P, _P,
        _P, _P, _P, c_int64, _P, c_int32,
        _P, _P, c_int64,
        _P, _P, c_int64,
        _P, _P, _P, _P,
        c_int32, c_int32,
        c_int32, c_int32, c_int32, c_int32, c_int32,
        c_float, c_int32,
        _P, c_int64, _P]),
    "tierkv_decode_attention_noalloc": (c_int32, [
        _P, c_int32, _P, _P,
        _P, _P, _P, c_int64, _P, c_int32,
        _P, _P, c_int64,
        _P, _P, c_int64,
        _P, _P, _P, _P,
        c_int32, c_int32,
        c_int32, c_int32, c_int32, c_int32, c_int32,
        c_float, c_int32, _P]),
    "tierkv_decode_workspace_bytes": (c_int64, [c_int32] * 8),
    "tierkv_decode_noalloc_error_word": (c_int32, [c_int32, _P]),
    "tierkv_demote_to_warm": (c_int32, [
        _P, _P, c_int64,
        _P, _P, _P, c_int32,
        _P, _P, c_int64,
        _P, _P, _P, _P,
        c_int32, c_int32,
        _P, _P, _P,
        c_int32, c_int32, c_int32, _P]),
    "tierkv_promote_to_hot": (c_int32, [
        _P, _P, c_int64,
        _P, _P, _P, _P,
        _P, _P, _P, c_int32,
        _P, _P, c_int64, c_int32,
        _P, _P, _P,
        c_int32, c_int32, c_int32, _P]),
    "tierkv_write_hot_tokens": (c_int32, [
        _P, _P, c_int64, c_int32,
        _P, _P, _P,
        _P, _P, c_int32, c_int32,
        _P, _P, c_int64,
        c_int32, c_int32, c_int32, _P]),
    "tierkv_runtime_append": (c_int32, [
        _P, _P, c_int32,
        _P, _P, _P, c_int64,
        _P, _P, c_int32, c_int32,
        _P, _P, c_int64, _P, _P,
        c_int32, c_int32, c_int32, _P]),
    "tierkv_runtime_append_rope": (c_int32, [
        _P, c_int64, c_int64, c_int64, c_int32, _P,
        _P, c_int64, c_int64, c_int64,
        _P, c_int64, c_int64, c_int64,
        _P, _P, c_int64, c_int64, c_int32,
        _P, _P, _P, c_int64,
        _P, _P, c_int32, c_int32,
        _P, _P, c_int64, _P, _P,
        c_int32, c_int32, c_int32, _P]),
    "tierkv_runtime_tick": (c_int32, [
        _P, c_int64, c_int32,
        _P, _P, _P, c_int64,
        _P, c_int32, c_int32, c_int32, c_int32,
        _P, _P, c_int64, _P,
        _P, _P, c_int64, _P,
        _P, _P, _P, _P, c_int32,
        _P, _P, c_int64, c_int32, c_int32,
        c_int32, c_int32, c_int32, _P]),
    "tierkv_runtime_tick_scratch_bytes": (c_int64, [c_int32, c_int64, c_int32, c_int32]),
    "tierkv_scatter_i32": (c_int32, [_P, c_int64, _P, c_int32, _P]),
    "tierkv_tier_counts": (c_int32, [_P, _P, c_int64, _P, c_int32, _P, _P]),
    "tierkv_scatter_i32_inline": (c_int32, [_P, c_int64, _P, c_int32, _P]),
    "tierkv_decode_step": (c_int32, [_P, _P]),
    "tierkv_decode_step_size": (c_int64, []),
    "tierkv_write_hot_tokens_inline": (c_int32, [
        _P, _P, c_int64, c_int32, _P, c_int32,
        c_int32, _P, _P, c_int64,
        c_int32, c_int32, c_int32, _P]),
    "tierkv_prefill_block_mass_workspace_bytes": (c_int64, [c_int32, c_int32, c_int32]),
    "tierkv_prefill_block_mass": (c_int32, [
        _P, c_int64, c_int64, c_int64,
        _P, c_int64, c_int64, c_int64, c_int32,
        _P, c_int32, c_int32, c_int32, c_int32, c_int32,
        c_int32, c_float, _P, c_int64, _P]),
    "tierkv_block_mass_from_probs": (c_int32, [_P, _P, _P, c_int32, c_int32, c_int32, c_int32, _P]),
    "tierkv_block_scores_from_sums": (c_int32, [_P, c_int64, _P, c_int64, _P, c_int32, c_int32, c_int32, _P]),
    "tierkv_tier_labels": (c_int32, [_P, _P, _P, c_int64, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, _P]),
    "tierkv_bm_create": (c_int32, [c_int32, POINTER(c_void_p)]),
    "tierkv_bm_destroy": (None, [_P]),
    "tierkv_bm_allocate_block": (c_int32, [_P, c_int32, _I32P]),
    "tierkv_bm_free_sequence": (c_int32, [_P, c_int32]),
    "tierkv_bm_update_block_state": (c_int32, [_P, c_int32, c_int32, c_int32]),
    "tierkv_bm_set_block_states": (c_int32, [_P, c_int32, _I32P, c_int32]),
    "tierkv_bm_num_blocks": (c_int32, [_P, c_int32, _I32P]),
    "tierkv_bm_get_physical_indices": (c_int32, [_P, c_int32, _I32P, c_int32, _I32P]),
    "tierkv_bm_get_states": (c_int32, [_P, c_int32, _I32P, c_int32, _I32P]),
    "tierkv_bm_num_free": (c_int32, [_P, _I32P]),
}

_lock = threading.Lock()
_lib = None


def lib():
    """The loaded library (RuntimeError if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH.name} is not built: run `python -m paged_tierkv_amd.build` "
                    "(the HIP path has no fallback).")
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            version = handle.tierkv_abi_version()
            if version != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH.name} ABI version {version} != expected {ABI_VERSION}; rebuild it.")
            if handle.tierkv_decode_step_size() != ctypes.sizeof(DecodeStep):
                raise RuntimeError(f"{LIB_PATH.name}: TierkvDecodeStep is {handle.tierkv_decode_step_size()} bytes, "
                                   f"the binding's {ctypes.sizeof(DecodeStep)}; rebuild it.")
            _lib = handle
    return _lib


def last_error() -> str:
    return lib().tierkv_last_error().decode("utf-8", "replace")


def check(rc: int, what: str = "") -> None:
    if rc == TIERKV_OK:
        return
    msg = last_error() or f"{what} failed with status {rc}"
    if rc == TIERKV_ERR_INVALID:
        raise ValueError(msg)
    raise RuntimeError(msg)


def ptr(t) -> int | None:
    """Device (or host) address of a tensor, None for None."""
    if t is None:
        return None
    return t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device) -> int:
    """Handle of torch's current stream on ``device`` (launches go there)."""
    if _raw_stream is not None:
        idx = device.index if isinstance(device, torch.device) else None
        return _raw_stream(torch.cuda.current_device() if idx is None else idx)
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu_tensor(t, name: str) -> None:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{name} must be a GPU (HIP) tensor.")


def library_exists() -> bool:
    return LIB_PATH.exists()


def env_flag(name: str) -> bool:
    return os.environ.get(name, "0").lower() in ("1", "true", "yes", "on")

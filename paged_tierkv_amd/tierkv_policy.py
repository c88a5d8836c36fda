"""Tier engine on MI355X -- drop-in for the reference module tierkv_policy.

Same public names, constructor arguments, return values and exceptions as
tierkv_policy.py: the codec pair (21-44), the dense ``TieredKVTensorPool``
(53-698, alias ``PhysicalKVPool``), ``CompactTieredKVTensorPool`` (701-1365),
``TierKVPolicyEngine`` (1372-1478), ``LayerRuntimeState`` (1481-1484), the
HF ``TieredKVCache`` (1487-1531), ``TieredKVRuntime`` (1534-1912) and the
module functions (1915-2044).  Host bookkeeping follows the reference rule
for rule -- BlockManager calls, LIFO free-slot lists refilled
``range(new - 1, old - 1, -1)``, slot and state transitions, error types and
messages -- so slot ids, tables and pool bytes come out identical.

What differs is how the device work is issued:

* every data movement runs in the HIP kernels of libtierkv_hip.so (token
  copies with tail zeroing, reference-codec quantize and dequantize); the
  module never falls back to PyTorch arithmetic, and a missing library raises
  RuntimeError;
* pool operations queue their copies and launch them in batches: a whole
  prefill is one copy launch plus one quantize launch, a whole
  ``sync_storage_states`` one demote and one promote launch, where the
  reference issues about 20 launches per block.  Queued jobs never overlap on
  a slot (a job that would read or write a slot a queued job writes, or write
  a slot a queued job reads, first launches the queue), so batching preserves
  the reference's sequential order;
* the block tables keep a host copy; entry writes are queued and pushed with
  one scatter launch when a table is next read (``get_layer_table``,
  ``get_layer_lengths`` or the table attributes), instead of one launch per
  entry; host-side reads (lengths, metrics) use the host copy, so
  ``collect_memory_metrics`` does not synchronise;
* the policy's ranking runs in the label kernel (one device-to-host copy per
  enforce call instead of one per candidate, tierkv_policy.py:1424, 1462).

Extension (keyword-only): ``warm_format="absmax_i8"`` stores WARM blocks as
int8 codes with fp32 per-(slot, head) scales (``k_zero``/``v_zero`` None);
the default ``"ref_u8"`` is the reference codec.

All tensors are GPU tensors; operations run on the current stream, which must
stay the same across calls on one device.
"""

from __future__ import annotations

import contextlib
import os
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from ._staging import stage_i32
from .kernels import LABEL_MODES, WARM_FORMATS

_INLINE_JOBS = 4     # copy jobs the inline write entry point carries (tierkv_write_hot_tokens_inline)
_INLINE_PAIRS = 16   # table writes the inline scatter carries (tierkv_scatter_i32_inline)

try:
    from transformers.cache_utils import Cache as HFCache
except Exception:  # transformers absent: the cache is a plain object, as in the reference
    HFCache = object


HOT_STATE = 0
WARM_STATE = 1
COLD_STATE = 2

_GLOBAL_TIERKV_RUNTIME = None


def _ceil_div(value: int, divisor: int) -> int:
    return (int(value) + int(divisor) - 1) // int(divisor)


def estimate_pool_blocks(num_layers: int, block_size: int, max_seq_len: int) -> int:
    return int(num_layers) * _ceil_div(max_seq_len, block_size)


def _ptr_at(t: torch.Tensor, offset: int) -> int:
    return t.data_ptr() + offset * t.element_size()


# ---------------------------------------------------------------------------
# Codec (tierkv_policy.py:21-44) on the GPU.
# ---------------------------------------------------------------------------

def _rows_as_tiles(x: torch.Tensor, rows: int, width: int):
    tiles = _ceil_div(max(rows, 1), 16)
    buf = torch.zeros((tiles * 16, width), dtype=x.dtype, device=x.device)
    buf[:rows].copy_(x.reshape(rows, width))
    return buf.view(tiles, 1, 16, width), tiles


def quantize_fp16_to_int8(tensor: torch.Tensor):
    """Per-row asymmetric uint8 codec over the last dim (tierkv_policy.py:21-36):
    returns (codes uint8, scale fp16 [..., 1], zero_point fp16 [..., 1]),
    bit-exact with the reference's fp16 op sequence."""
    lib = _lib.lib()
    _lib.require_gpu_tensor(tensor, "tensor")
    if tensor.dtype != torch.float16:
        tensor = tensor.to(torch.float16)
    shape = tuple(tensor.shape)
    dim = int(shape[-1])
    rows = tensor.numel() // max(dim, 1)
    src, tiles = _rows_as_tiles(tensor.contiguous(), rows, dim)
    codes = torch.empty((tiles, 1, 16, dim), dtype=torch.uint8, device=tensor.device)
    scale = torch.empty((tiles, 1, 16, 1), dtype=torch.float16, device=tensor.device)
    zero = torch.empty_like(scale)
    codes_v, scale_v, zero_v = torch.empty_like(codes), torch.empty_like(scale), torch.empty_like(scale)
    jobs = np.concatenate([np.arange(tiles), np.arange(tiles), np.full(tiles, 16)]).astype(np.int32)
    jobs[3 * tiles - 1] = rows - 16 * (tiles - 1)
    d = stage_i32(jobs, tensor.device)
    rc = lib.tierkv_demote_to_warm(
        _lib.ptr(src), _lib.ptr(src), tiles,
        _ptr_at(d, 0), _ptr_at(d, tiles), _ptr_at(d, 2 * tiles), tiles,
        _lib.ptr(codes), _lib.ptr(codes_v), tiles,
        _lib.ptr(scale), _lib.ptr(zero), _lib.ptr(scale_v), _lib.ptr(zero_v),
        _lib.WARM_REF_U8, 1, None, None, None, 1, 16, dim, _lib.stream_of(tensor.device))
    _lib.check(rc, "quantize_fp16_to_int8")
    meta_shape = shape[:-1] + (1,)
    return (codes.view(-1, dim)[:rows].reshape(shape), scale.view(-1)[:rows].reshape(meta_shape),
            zero.view(-1)[:rows].reshape(meta_shape))


def dequantize_int8_to_fp16(quantized_tensor: torch.Tensor, scale: torch.Tensor, zero_point: torch.Tensor):
    """((q.to(fp16) - zero_point) * scale).to(fp16) per row (tierkv_policy.py:39-44)."""
    lib = _lib.lib()
    for name, t in (("quantized_tensor", quantized_tensor), ("scale", scale), ("zero_point", zero_point)):
        _lib.require_gpu_tensor(t, name)
    if quantized_tensor.dtype != torch.uint8:
        raise ValueError("quantized_tensor must be uint8.")
    shape = tuple(quantized_tensor.shape)
    dim = int(shape[-1])
    rows = quantized_tensor.numel() // max(dim, 1)
    meta_shape = shape[:-1] + (1,)
    sc = scale.to(torch.float16).expand(meta_shape).contiguous()
    zp = zero_point.to(torch.float16).expand(meta_shape).contiguous()
    codes, tiles = _rows_as_tiles(quantized_tensor.contiguous(), rows, dim)
    sc_t, _ = _rows_as_tiles(sc, rows, 1)
    zp_t, _ = _rows_as_tiles(zp, rows, 1)
    out = torch.empty((tiles, 1, 16, dim), dtype=torch.float16, device=quantized_tensor.device)
    out_v = torch.empty_like(out)
    jobs = np.concatenate([np.arange(tiles), np.arange(tiles), np.full(tiles, 16)]).astype(np.int32)
    jobs[3 * tiles - 1] = rows - 16 * (tiles - 1)
    d = stage_i32(jobs, quantized_tensor.device)
    rc = lib.tierkv_promote_to_hot(
        _lib.ptr(codes), _lib.ptr(codes), tiles,
        _lib.ptr(sc_t), _lib.ptr(zp_t), _lib.ptr(sc_t), _lib.ptr(zp_t),
        _ptr_at(d, 0), _ptr_at(d, tiles), _ptr_at(d, 2 * tiles), tiles,
        _lib.ptr(out), _lib.ptr(out_v), tiles, _lib.WARM_REF_U8,
        None, None, None, 1, 16, dim, _lib.stream_of(quantized_tensor.device))
    _lib.check(rc, "dequantize_int8_to_fp16")
    return out.view(-1, dim)[:rows].reshape(shape)


# ---------------------------------------------------------------------------
# Device tables with a host copy.
# ---------------------------------------------------------------------------

class _Tables:
    """int32 tables [num_layers, max_blocks] packed as one device tensor
    [num_layers, k, max_blocks] with a host copy.  Writes update the host copy
    and queue the entry; ``flush`` pushes the queue with one scatter launch."""

    def __init__(self, fills, num_layers: int, max_blocks: int, device):
        self.fills = list(fills)
        k = len(self.fills)
        self.shape = (int(num_layers), k, int(max_blocks))
        self.host = np.empty(self.shape, np.int32)
        for i, f in enumerate(self.fills):
            self.host[:, i, :] = f
        self.dev = torch.empty(self.shape, dtype=torch.int32, device=device)
        for i, f in enumerate(self.fills):
            self.dev[:, i, :].fill_(f)
        self.pending: dict[int, int] = {}

    def _flat(self, k: int, layer: int, idx: int) -> int:
        return (layer * self.shape[1] + k) * self.shape[2] + idx

    def set(self, k: int, layer: int, idx: int, value: int) -> None:
        layer, idx, value = int(layer), int(idx), int(value)
        if not (0 <= layer < self.shape[0]):
            raise IndexError(f"index {layer} is out of bounds for dimension 0 with size {self.shape[0]}")
        if not (-self.shape[2] <= idx < self.shape[2]):
            raise IndexError(f"index {idx} is out of bounds for dimension 1 with size {self.shape[2]}")
        idx %= self.shape[2]
        self.host[layer, k, idx] = value
        self.pending[self._flat(k, layer, idx)] = value

    def get(self, k: int, layer: int, idx: int) -> int:
        return int(self.host[int(layer), k, int(idx)])

    def row(self, k: int, layer: int) -> np.ndarray:
        return self.host[int(layer), k]

    def fill_row(self, k: int, layer: int, value: int) -> None:
        layer = int(layer)
        self.host[layer, k, :] = value
        base = self._flat(k, layer, 0)
        for i in range(self.shape[2]):
            self.pending[base + i] = int(value)

    def reset(self) -> None:
        self.pending.clear()
        for i, f in enumerate(self.fills):
            self.host[:, i, :] = f
            self.dev[:, i, :].fill_(f)

    def flush(self) -> None:
        if not self.pending:
            return
        n = len(self.pending)
        pairs = np.fromiter((x for kv in self.pending.items() for x in kv), dtype=np.int32, count=2 * n)
        self.pending.clear()
        _scatter(self.dev, pairs, n)

    def view(self, k: int) -> torch.Tensor:
        self.flush()
        return self.dev[:, k, :]


def _scatter(dev: torch.Tensor, pairs: np.ndarray, n: int) -> None:
    """dev[pairs[2i]] = pairs[2i + 1]: up to 16 pairs ride in the kernel's
    arguments, more go through the pinned staging ring."""
    lib = _lib.lib()
    stream = _lib.stream_of(dev.device)
    if n <= _INLINE_PAIRS:
        rc = lib.tierkv_scatter_i32_inline(_lib.ptr(dev), dev.numel(), pairs.ctypes.data, n, stream)
        _lib.check(rc, "tierkv_scatter_i32_inline")
        return
    d = stage_i32(pairs, dev.device)
    rc = lib.tierkv_scatter_i32(_lib.ptr(dev), dev.numel(), _lib.ptr(d), n, stream)
    _lib.check(rc, "tierkv_scatter_i32")


class _Vector:
    """Growable int32 device vector with a host copy (the dense pool's
    per-physical-block lengths)."""

    def __init__(self, capacity: int, device):
        self.host = np.zeros(int(capacity), np.int32)
        self.dev = torch.zeros(int(capacity), dtype=torch.int32, device=device)
        self.pending: dict[int, int] = {}

    def grow(self, capacity: int) -> None:
        self.flush()
        old = self.host.size
        host = np.zeros(int(capacity), np.int32)
        host[:old] = self.host
        dev = torch.zeros(int(capacity), dtype=torch.int32, device=self.dev.device)
        dev[:old].copy_(self.dev[:old])
        self.host, self.dev = host, dev

    def set(self, idx: int, value: int) -> None:
        idx = int(idx)
        if not (-self.host.size <= idx < self.host.size):
            raise IndexError(f"index {idx} is out of bounds for dimension 0 with size {self.host.size}")
        idx %= self.host.size
        self.host[idx] = int(value)
        self.pending[idx] = int(value)

    def zero(self) -> None:
        self.pending.clear()
        self.host[:] = 0
        self.dev.zero_()

    def flush(self) -> None:
        if not self.pending:
            return
        n = len(self.pending)
        pairs = np.fromiter((x for kv in self.pending.items() for x in kv), dtype=np.int32, count=2 * n)
        self.pending.clear()
        _scatter(self.dev, pairs, n)

    def tensor(self) -> torch.Tensor:
        self.flush()
        return self.dev


# ---------------------------------------------------------------------------
# Shared storage machinery: queued data movement.
# ---------------------------------------------------------------------------

class _QueuedStorage:
    """Queue of data movement between pools, launched in conflict-free batches.

    Job kinds (slots are HOT-pool / WARM-pool slot indices):
      write  -- tokens of an external fp16 source into a HOT slot (tail zeroed)
      stage  -- tokens of an external fp16 source quantized into a WARM slot
      demote -- HOT slot quantized into a WARM slot
      promote-- WARM slot dequantized into a HOT slot
    """

    _demote_pads_tail = False      # compact demote_to_warm leaves the WARM tail as it was
    _stage_pads_tail = True        # compact write_warm_block pads the tail

    def _init_queue(self) -> None:
        self._depth = 0
        self._reset_queue()

    def _reset_queue(self) -> None:
        self._q_write: list = []
        self._q_stage: list = []
        self._q_dem: list = []
        self._q_pro: list = []
        self._r_hot: set = set()
        self._w_hot: set = set()
        self._r_warm: set = set()
        self._w_warm: set = set()

    @contextlib.contextmanager
    def _batch(self):
        self._depth += 1
        try:
            yield
        finally:
            # Launch even when the operation raised part-way: the host state
            # already records the writes planned before the error, as the
            # reference has already executed them.
            self._depth -= 1
            if self._depth == 0:
                self._launch_queue()

    def _touch(self, r_hot=(), w_hot=(), r_warm=(), w_warm=()) -> None:
        conflict = (any(s in self._w_hot for s in r_hot)
                    or any(s in self._w_hot or s in self._r_hot for s in w_hot)
                    or any(s in self._w_warm for s in r_warm)
                    or any(s in self._w_warm or s in self._r_warm for s in w_warm))
        if conflict:
            self._launch_queue()
        self._r_hot.update(r_hot)
        self._w_hot.update(w_hot)
        self._r_warm.update(r_warm)
        self._w_warm.update(w_warm)

    def _queue_write(self, src_k, src_v, tok0: int, count: int, hot_slot: int, pos: int) -> None:
        self._touch(w_hot=(hot_slot,))
        self._q_write.append((src_k, src_v, int(tok0), int(count), int(hot_slot), int(pos)))
        if self._depth == 0:
            self._launch_queue()

    def _queue_stage(self, src_k, src_v, tok0: int, count: int, warm_slot: int) -> None:
        self._touch(w_warm=(warm_slot,))
        self._q_stage.append((src_k, src_v, int(tok0), int(count), int(warm_slot)))
        if self._depth == 0:
            self._launch_queue()

    def _queue_demote(self, hot_slot: int, warm_slot: int, length: int) -> None:
        self._touch(r_hot=(hot_slot,), w_warm=(warm_slot,))
        self._q_dem.append((int(hot_slot), int(warm_slot), int(length)))
        if self._depth == 0:
            self._launch_queue()

    def _queue_promote(self, warm_slot: int, hot_slot: int, length: int) -> None:
        self._touch(r_warm=(warm_slot,), w_hot=(hot_slot,))
        self._q_pro.append((int(warm_slot), int(hot_slot), int(length)))
        if self._depth == 0:
            self._launch_queue()

    @staticmethod
    def _group_by_source(jobs):
        groups: dict = {}
        for job in jobs:
            key = (id(job[0]), id(job[1]))
            groups.setdefault(key, (job[0], job[1], []))[2].append(job[2:])
        return groups.values()

    def _launch_writes(self, lib, src_k, src_v, rows, dst_k, dst_v, stream) -> None:
        n = len(rows)
        if n <= _INLINE_JOBS:
            # A decode step's few jobs ride in the kernel's arguments.
            jobs = np.zeros((n, 5), np.int32)     # src_seq, src_tok, count, dst_slot, dst_pos
            for i, (tok0, count, slot, pos) in enumerate(rows):
                jobs[i, 1], jobs[i, 2], jobs[i, 3], jobs[i, 4] = tok0, count, slot, pos
            rc = lib.tierkv_write_hot_tokens_inline(
                _lib.ptr(src_k), _lib.ptr(src_v), int(src_k.shape[0]), int(src_k.shape[2]), jobs.ctypes.data, n, 1,
                _lib.ptr(dst_k), _lib.ptr(dst_v), int(dst_k.shape[0]),
                self.kv_heads, self.block_size, self.head_dim, stream)
            _lib.check(rc, "tierkv_write_hot_tokens_inline")
            return
        arr = np.zeros((5, n), np.int32)          # src_seq, src_tok, count, dst_slot, dst_pos
        for i, (tok0, count, slot, pos) in enumerate(rows):
            arr[1, i], arr[2, i], arr[3, i], arr[4, i] = tok0, count, slot, pos
        d = stage_i32(arr, src_k.device)
        rc = lib.tierkv_write_hot_tokens(
            _lib.ptr(src_k), _lib.ptr(src_v), int(src_k.shape[0]), int(src_k.shape[2]),
            _ptr_at(d, 0), _ptr_at(d, n), _ptr_at(d, 2 * n), _ptr_at(d, 3 * n), _ptr_at(d, 4 * n), n, 1,
            _lib.ptr(dst_k), _lib.ptr(dst_v), int(dst_k.shape[0]),
            self.kv_heads, self.block_size, self.head_dim, stream)
        _lib.check(rc, "tierkv_write_hot_tokens")

    def _launch_quantize(self, lib, src_k, src_v, src_idx, dst, lengths, pad_tail, stream) -> None:
        n = len(src_idx)
        d = stage_i32(np.asarray([src_idx, dst, lengths], np.int32), src_k.device)
        rc = lib.tierkv_demote_to_warm(
            _lib.ptr(src_k), _lib.ptr(src_v), int(src_k.shape[0]),
            _ptr_at(d, 0), _ptr_at(d, n), _ptr_at(d, 2 * n), n,
            _lib.ptr(self.warm_k_pool), _lib.ptr(self.warm_v_pool), int(self.warm_k_pool.shape[0]),
            _lib.ptr(self.k_scale), _lib.ptr(self.k_zero), _lib.ptr(self.v_scale), _lib.ptr(self.v_zero),
            WARM_FORMATS[self.warm_format], int(pad_tail), None, None, None,
            self.kv_heads, self.block_size, self.head_dim, stream)
        _lib.check(rc, "tierkv_demote_to_warm")

    def _launch_dequantize(self, lib, src, dst, lengths, dst_k, dst_v, stream) -> None:
        n = len(src)
        d = stage_i32(np.asarray([src, dst, lengths], np.int32), dst_k.device)
        rc = lib.tierkv_promote_to_hot(
            _lib.ptr(self.warm_k_pool), _lib.ptr(self.warm_v_pool), int(self.warm_k_pool.shape[0]),
            _lib.ptr(self.k_scale), _lib.ptr(self.k_zero), _lib.ptr(self.v_scale), _lib.ptr(self.v_zero),
            _ptr_at(d, 0), _ptr_at(d, n), _ptr_at(d, 2 * n), n,
            _lib.ptr(dst_k), _lib.ptr(dst_v), int(dst_k.shape[0]), WARM_FORMATS[self.warm_format],
            None, None, None, self.kv_heads, self.block_size, self.head_dim, stream)
        _lib.check(rc, "tierkv_promote_to_hot")

    def _launch_queue(self) -> None:
        if not (self._q_write or self._q_stage or self._q_dem or self._q_pro):
            self._reset_queue()
            return
        lib = _lib.lib()
        stream = _lib.stream_of(self.device)
        writes, stages, dems, pros = self._q_write, self._q_stage, self._q_dem, self._q_pro
        self._reset_queue()
        for src_k, src_v, rows in self._group_by_source(writes):
            self._launch_writes(lib, src_k, src_v, rows, self.hot_k_pool, self.hot_v_pool, stream)
        for src_k, src_v, rows in self._group_by_source(stages):
            tiles = torch.empty((len(rows), self.kv_heads, self.block_size, self.head_dim),
                                dtype=torch.float16, device=self.device)
            tiles_v = torch.empty_like(tiles)
            self._launch_writes(lib, src_k, src_v, [(t0, c, i, 0) for i, (t0, c, _) in enumerate(rows)],
                                tiles, tiles_v, stream)
            self._launch_quantize(lib, tiles, tiles_v, list(range(len(rows))), [r[2] for r in rows],
                                  [r[1] for r in rows], self._stage_pads_tail, stream)
        if dems:
            self._launch_quantize(lib, self.hot_k_pool, self.hot_v_pool, [j[0] for j in dems],
                                  [j[1] for j in dems], [j[2] for j in dems], self._demote_pads_tail, stream)
        if pros:
            self._launch_dequantize(lib, [j[0] for j in pros], [j[1] for j in pros], [j[2] for j in pros],
                                    self.hot_k_pool, self.hot_v_pool, stream)

    def _dequantize_slot(self, warm_slot: int, length: int):
        """fp16 K, V [1, kv_heads, length, head_dim] of one WARM slot."""
        self._launch_queue()
        tile_k = torch.zeros((1, self.kv_heads, self.block_size, self.head_dim), dtype=torch.float16,
                             device=self.device)
        tile_v = torch.zeros_like(tile_k)
        self._launch_dequantize(_lib.lib(), [warm_slot], [0], [length], tile_k, tile_v,
                                _lib.stream_of(self.device))
        return tile_k[:, :, :length, :].contiguous(), tile_v[:, :, :length, :].contiguous()

    # -- WARM pools in either format ---------------------------------------
    def _check_format(self, warm_format: str) -> str:
        if warm_format not in WARM_FORMATS:
            raise ValueError('warm_format must be "ref_u8" or "absmax_i8".')
        return warm_format

    def _warm_dtype(self):
        return torch.uint8 if self.warm_format == "ref_u8" else torch.int8

    def _new_scale(self, capacity: int, fill):
        if self.warm_format == "ref_u8":
            return torch.full((capacity, self.kv_heads, self.block_size, 1), fill, device=self.device,
                              dtype=torch.float16)
        return torch.zeros((capacity, self.kv_heads), device=self.device, dtype=torch.float32)

    def _new_zero_point(self, capacity: int):
        if self.warm_format == "ref_u8":
            return torch.zeros((capacity, self.kv_heads, self.block_size, 1), device=self.device,
                               dtype=torch.float16)
        return None

    @staticmethod
    def _grow_copy(old, new, old_capacity: int):
        if old is not None and new is not None and old_capacity > 0:
            new[:old_capacity].copy_(old[:old_capacity])
        return new

    @staticmethod
    def _source(key_states: torch.Tensor, value_states: torch.Tensor):
        """Whole [1, kv_heads, T, head_dim] fp16 sources for range writes."""
        if key_states.shape != value_states.shape:
            raise ValueError("Key and value tensors must have identical shape.")
        if key_states.ndim != 4 or key_states.shape[0] != 1:
            raise ValueError("KV tensors must have shape [1, kv_heads, tokens, head_dim].")
        _lib.require_gpu_tensor(key_states, "key_states")
        _lib.require_gpu_tensor(value_states, "value_states")
        if key_states.dtype != torch.float16:
            key_states = key_states.to(torch.float16)
        if value_states.dtype != torch.float16:
            value_states = value_states.to(torch.float16)
        return key_states.contiguous(), value_states.contiguous()

    def _coerce_kv(self, key_states: torch.Tensor, value_states: torch.Tensor):
        if key_states.shape != value_states.shape:
            raise ValueError("Key and value tensors must have identical shape.")
        if key_states.ndim != 4 or key_states.shape[0] != 1:
            raise ValueError("KV tensors must have shape [1, kv_heads, tokens, head_dim].")
        if key_states.shape[-2] > self.block_size:
            raise ValueError("A single stored block cannot exceed block_size tokens.")
        return self._source(key_states, value_states)

    @staticmethod
    def _tensor_mb(tensor: torch.Tensor | None) -> float:
        if tensor is None:
            return 0.0
        return tensor.numel() * tensor.element_size() / (1024 ** 2)

    def _warm_token_meta_bytes(self) -> int:
        return int(self.kv_heads) * 4 * 2


def _zero_metrics() -> dict:
    return {
        "hot_blocks": 0, "warm_blocks": 0, "cold_blocks": 0,
        "hot_tokens": 0, "warm_tokens": 0, "cold_tokens": 0, "active_tokens": 0,
        "logical_hot_mb": 0.0, "logical_warm_mb": 0.0, "logical_warm_meta_mb": 0.0,
        "logical_cold_evicted_mb": 0.0, "logical_dense_equivalent_mb": 0.0, "logical_resident_mb": 0.0,
        "logical_compression_ratio": 0.0, "logical_compression_x": 0.0,
    }


def _logical_metrics(kv_heads, head_dim, hot_tokens, warm_tokens, cold_tokens, meta_bytes_per_token):
    """Byte accounting of collect_memory_metrics (tierkv_policy.py:586-609,
    1263-1276): fp16 K+V per HOT/COLD token, int8 K+V per WARM token plus
    the per-token metadata."""
    dense_tok = kv_heads * head_dim * 2 * 2
    int8_tok = kv_heads * head_dim * 2
    active = hot_tokens + warm_tokens + cold_tokens
    hot_b = hot_tokens * dense_tok
    warm_b = warm_tokens * int8_tok
    meta_b = warm_tokens * meta_bytes_per_token
    cold_b = cold_tokens * dense_tok
    dense_b = active * dense_tok
    resident_b = hot_b + warm_b + meta_b
    mb = 1024 ** 2
    return {
        "active_tokens": active,
        "logical_hot_mb": hot_b / mb,
        "logical_warm_mb": warm_b / mb,
        "logical_warm_meta_mb": meta_b / mb,
        "logical_cold_evicted_mb": cold_b / mb,
        "logical_dense_equivalent_mb": dense_b / mb,
        "logical_resident_mb": resident_b / mb,
        "_dense_b": dense_b,
        "_resident_b": resident_b,
    }


# ---------------------------------------------------------------------------
# Dense pool (tierkv_policy.py:53-698): one storage row per physical block in
# every pool; tables hold the physical id.
# ---------------------------------------------------------------------------

class TieredKVTensorPool(_QueuedStorage):
    _demote_pads_tail = True       # dense demote_to_warm zero-pads (350-356)
    _stage_pads_tail = False       # dense write_warm_block copies [:length] only (292-312)

    _T_TABLE, _T_STATE, _T_LEN = 0, 1, 2

    def __init__(
        self,
        num_layers: int = 1,
        block_size: int = 16,
        max_seq_len: int = 2048,
        max_blocks_per_layer: int | None = None,
        pool_blocks: int | None = None,
        pool_chunk_blocks: int = 128,
        *,
        warm_format: str = "ref_u8",
    ):
        if num_layers <= 0:
            raise ValueError("num_layers must be positive.")
        if block_size <= 0:
            raise ValueError("block_size must be positive.")
        if max_seq_len <= 0:
            raise ValueError("max_seq_len must be positive.")

        self.num_layers = int(num_layers)
        self.block_size = int(block_size)
        self.max_seq_len = int(max_seq_len)
        self.max_blocks_per_layer = int(max_blocks_per_layer or _ceil_div(max_seq_len, block_size))
        self.pool_blocks = int(pool_blocks or self.num_layers * self.max_blocks_per_layer)
        self.pool_chunk_blocks = int(pool_chunk_blocks)
        if self.pool_chunk_blocks <= 0:
            raise ValueError("pool_chunk_blocks must be positive.")
        self.warm_format = self._check_format(warm_format)

        self.device = None
        self.dtype = torch.float16
        self.kv_heads = None
        self.head_dim = None
        self.allocated_pool_blocks = 0

        self.hot_k_pool = None
        self.hot_v_pool = None
        self.warm_k_pool = None
        self.warm_v_pool = None
        self.k_scale = None
        self.k_zero = None
        self.v_scale = None
        self.v_zero = None
        self._lengths: _Vector | None = None        # per physical block (block_lengths)
        self._tables: _Tables | None = None         # block_tables, block_states, logical_block_lengths
        self.full_table_sync_count = 0

        self.physical_states: dict[int, int] = {}
        self.physical_locations: dict[int, tuple[int, int]] = {}
        self.hot_storage = set()
        self.warm_storage = set()
        self.cold_storage = set()
        self._init_queue()

    # Device views of the tables (queued entries pushed first).
    @property
    def block_lengths(self):
        return None if self._lengths is None else self._lengths.tensor()

    @property
    def block_tables(self):
        return None if self._tables is None else self._tables.view(self._T_TABLE)

    @property
    def block_states(self):
        return None if self._tables is None else self._tables.view(self._T_STATE)

    @property
    def logical_block_lengths(self):
        return None if self._tables is None else self._tables.view(self._T_LEN)

    def is_allocated(self) -> bool:
        return self.hot_k_pool is not None

    def _target_capacity(self, physical_idx: int) -> int:
        required = int(physical_idx) + 1
        return min(self.pool_blocks, _ceil_div(required, self.pool_chunk_blocks) * self.pool_chunk_blocks)

    def _check_physical_idx(self, physical_idx: int) -> int:
        physical_idx = int(physical_idx)
        if physical_idx < 0 or physical_idx >= self.pool_blocks:
            raise RuntimeError(
                f"Physical block {physical_idx} is outside tensor-pool capacity {self.pool_blocks}."
            )
        return physical_idx

    def _grow_storage(self, required_physical_idx: int) -> None:
        if required_physical_idx < self.allocated_pool_blocks:
            return
        new_capacity = self._target_capacity(required_physical_idx)
        if new_capacity <= self.allocated_pool_blocks:
            return
        old = self.allocated_pool_blocks
        self._launch_queue()
        shape = (new_capacity, self.kv_heads, self.block_size, self.head_dim)
        self.hot_k_pool = self._grow_copy(self.hot_k_pool, torch.zeros(shape, device=self.device,
                                                                      dtype=torch.float16), old)
        self.hot_v_pool = self._grow_copy(self.hot_v_pool, torch.zeros(shape, device=self.device,
                                                                      dtype=torch.float16), old)
        self.warm_k_pool = self._grow_copy(self.warm_k_pool, torch.zeros(shape, device=self.device,
                                                                        dtype=self._warm_dtype()), old)
        self.warm_v_pool = self._grow_copy(self.warm_v_pool, torch.zeros(shape, device=self.device,
                                                                        dtype=self._warm_dtype()), old)
        self.k_scale = self._grow_copy(self.k_scale, self._new_scale(new_capacity, 1), old)
        self.k_zero = self._grow_copy(self.k_zero, self._new_zero_point(new_capacity), old)
        self.v_scale = self._grow_copy(self.v_scale, self._new_scale(new_capacity, 1), old)
        self.v_zero = self._grow_copy(self.v_zero, self._new_zero_point(new_capacity), old)
        if self._lengths is None:
            self._lengths = _Vector(new_capacity, self.device)
        else:
            self._lengths.grow(new_capacity)
        self.allocated_pool_blocks = new_capacity

    def _ensure_allocated(self, key_states: torch.Tensor, required_physical_idx: int) -> None:
        if key_states.ndim != 4:
            raise ValueError("KV tensors must have shape [1, kv_heads, tokens, head_dim].")
        if key_states.shape[0] != 1:
            raise ValueError("TieredKVTensorPool currently supports batch size 1 only.")
        device = key_states.device
        kv_heads = int(key_states.shape[1])
        head_dim = int(key_states.shape[-1])
        if self.is_allocated():
            if device != self.device or kv_heads != self.kv_heads or head_dim != self.head_dim:
                raise ValueError("KV tensor geometry changed after tensor-pool allocation.")
            self._grow_storage(required_physical_idx)
            return
        self.device = device
        self.kv_heads = kv_heads
        self.head_dim = head_dim
        self._tables = _Tables((-1, COLD_STATE, 0), self.num_layers, self.max_blocks_per_layer, device)
        self._grow_storage(required_physical_idx)

    def get_physical_state(self, physical_idx: int) -> int | None:
        return self.physical_states.get(int(physical_idx))

    def get_block_length(self, physical_idx: int) -> int:
        self._check_physical_idx(physical_idx)
        if self._lengths is None or int(physical_idx) >= self.allocated_pool_blocks:
            return 0
        return int(self._lengths.host[int(physical_idx)])

    def _note_length(self, physical_idx: int, length: int) -> None:
        self._lengths.set(physical_idx, length)
        if physical_idx in self.physical_locations and self._tables is not None:
            layer_idx, logical_idx = self.physical_locations[physical_idx]
            self._tables.set(self._T_LEN, layer_idx, logical_idx, length)

    def _write_hot_range(self, physical_idx, start, src_k, src_v, tok0, tokens) -> None:
        physical_idx = self._check_physical_idx(physical_idx)
        self._ensure_allocated(src_k, physical_idx)
        start, tokens = int(start), int(tokens)
        if start < 0 or start + tokens > self.block_size:
            raise ValueError("KV write exceeds the physical block capacity.")
        self._queue_write(src_k, src_v, tok0, tokens, physical_idx, start)
        self._note_length(physical_idx, start + tokens)
        self.physical_states[physical_idx] = HOT_STATE
        self.hot_storage.add(physical_idx)
        self.warm_storage.discard(physical_idx)
        self.cold_storage.discard(physical_idx)

    def write_hot_tokens(self, physical_idx: int, start: int, key_states: torch.Tensor,
                         value_states: torch.Tensor) -> None:
        """tierkv_policy.py:238-267."""
        physical_idx = self._check_physical_idx(physical_idx)
        key_states, value_states = self._coerce_kv(key_states, value_states)
        self._write_hot_range(physical_idx, start, key_states, value_states, 0, key_states.shape[-2])

    def set_block_entry(self, layer_idx: int, logical_idx: int, physical_idx: int, state: int) -> None:
        """tierkv_policy.py:269-285."""
        if not self.is_allocated():
            raise RuntimeError("TieredKVTensorPool has not been allocated yet.")
        layer_idx = int(layer_idx)
        logical_idx = int(logical_idx)
        physical_idx = self._check_physical_idx(physical_idx)
        if layer_idx < 0 or layer_idx >= self.num_layers:
            raise ValueError("layer_idx is out of range.")
        if logical_idx < 0 or logical_idx >= self.max_blocks_per_layer:
            raise RuntimeError(
                f"Logical block {logical_idx} exceeds max_blocks_per_layer={self.max_blocks_per_layer}."
            )
        if physical_idx >= self._lengths.host.size:
            raise IndexError(f"index {physical_idx} is out of bounds for dimension 0 with size "
                             f"{self._lengths.host.size}")
        self._tables.set(self._T_TABLE, layer_idx, logical_idx, physical_idx)
        self._tables.set(self._T_STATE, layer_idx, logical_idx, int(state))
        self._tables.set(self._T_LEN, layer_idx, logical_idx, int(self._lengths.host[physical_idx]))
        self.physical_locations[physical_idx] = (layer_idx, logical_idx)

    def set_block_state(self, layer_idx: int, logical_idx: int, state: int) -> None:
        if not self.is_allocated():
            raise RuntimeError("TieredKVTensorPool has not been allocated yet.")
        self._tables.set(self._T_STATE, layer_idx, logical_idx, int(state))

    def _write_warm_range(self, physical_idx, src_k, src_v, tok0, length) -> None:
        physical_idx = self._check_physical_idx(physical_idx)
        self._ensure_allocated(src_k, physical_idx)
        self._queue_stage(src_k, src_v, tok0, length, physical_idx)
        self._note_length(physical_idx, int(length))
        self.physical_states[physical_idx] = WARM_STATE
        self.hot_storage.discard(physical_idx)
        self.warm_storage.add(physical_idx)
        self.cold_storage.discard(physical_idx)

    def write_warm_block(self, physical_idx, k_tensor, v_tensor) -> None:
        """tierkv_policy.py:292-312 (tokens past the block's length untouched)."""
        physical_idx = self._check_physical_idx(physical_idx)
        k_tensor, v_tensor = self._coerce_kv(k_tensor, v_tensor)
        self._write_warm_range(physical_idx, k_tensor, v_tensor, 0, k_tensor.shape[-2])

    def register_cold_block(self, physical_idx, length: int) -> None:
        """tierkv_policy.py:314-324."""
        physical_idx = self._check_physical_idx(physical_idx)
        if self._lengths is not None:
            self._note_length(physical_idx, int(length))
        self.physical_states[physical_idx] = COLD_STATE
        self.hot_storage.discard(physical_idx)
        self.warm_storage.discard(physical_idx)
        self.cold_storage.add(physical_idx)

    def store_hot_block(self, physical_idx, k_tensor, v_tensor) -> None:
        self.write_hot_tokens(int(physical_idx), 0, k_tensor, v_tensor)

    def demote_to_warm(self, physical_idx) -> None:
        """tierkv_policy.py:329-361: quantize in place, tail zero-padded."""
        physical_idx = self._check_physical_idx(physical_idx)
        if self.get_physical_state(physical_idx) == WARM_STATE:
            return
        if self.get_physical_state(physical_idx) == COLD_STATE:
            raise KeyError(f"Physical block {physical_idx} is not eligible for WARM demotion from COLD storage.")
        if not self.is_allocated() or self.get_block_length(physical_idx) == 0:
            raise KeyError(f"Physical block {physical_idx} is not present in HOT storage.")
        self._queue_demote(physical_idx, physical_idx, self.get_block_length(physical_idx))
        self.physical_states[physical_idx] = WARM_STATE
        self.hot_storage.discard(physical_idx)
        self.warm_storage.add(physical_idx)
        self.cold_storage.discard(physical_idx)

    def demote_to_cold(self, physical_idx) -> None:
        """tierkv_policy.py:363-373 (metadata only)."""
        physical_idx = self._check_physical_idx(physical_idx)
        if self.get_physical_state(physical_idx) == COLD_STATE:
            return
        if not self.is_allocated() or self.get_block_length(physical_idx) == 0:
            raise KeyError(f"Physical block {physical_idx} is not present in HOT or WARM storage.")
        self.physical_states[physical_idx] = COLD_STATE
        self.hot_storage.discard(physical_idx)
        self.warm_storage.discard(physical_idx)
        self.cold_storage.add(physical_idx)

    def promote_to_hot(self, physical_idx) -> None:
        """tierkv_policy.py:375-402: dequantize [:length] in place."""
        physical_idx = self._check_physical_idx(physical_idx)
        state = self.get_physical_state(physical_idx)
        if state == HOT_STATE:
            return
        if state == COLD_STATE:
            raise KeyError(f"Physical block {physical_idx} is not eligible for HOT promotion from COLD storage.")
        if state != WARM_STATE:
            raise KeyError(f"Physical block {physical_idx} is not present in WARM storage.")
        self._queue_promote(physical_idx, physical_idx, self.get_block_length(physical_idx))
        self.physical_states[physical_idx] = HOT_STATE
        self.hot_storage.add(physical_idx)
        self.warm_storage.discard(physical_idx)
        self.cold_storage.discard(physical_idx)

    def get_dequantized_block(self, physical_idx, state):
        """tierkv_policy.py:404-448."""
        physical_idx = self._check_physical_idx(physical_idx)
        if not self.is_allocated():
            raise KeyError(f"Physical block {physical_idx} is not present in tensor-pool storage.")
        length = self.get_block_length(physical_idx)
        if state == HOT_STATE:
            if self.get_physical_state(physical_idx) == WARM_STATE:
                self.promote_to_hot(physical_idx)
            if self.get_physical_state(physical_idx) == COLD_STATE:
                raise KeyError(f"Physical block {physical_idx} is marked HOT but only exists in COLD storage.")
            self._launch_queue()
            return (self.hot_k_pool[physical_idx: physical_idx + 1, :, :length, :].contiguous(),
                    self.hot_v_pool[physical_idx: physical_idx + 1, :, :length, :].contiguous())
        if state == WARM_STATE:
            if self.get_physical_state(physical_idx) == COLD_STATE:
                raise KeyError(f"Physical block {physical_idx} is marked WARM but only exists in COLD storage.")
            self._launch_queue()
            if self.get_physical_state(physical_idx) == HOT_STATE:
                return (self.hot_k_pool[physical_idx: physical_idx + 1, :, :length, :].contiguous(),
                        self.hot_v_pool[physical_idx: physical_idx + 1, :, :length, :].contiguous())
            return self._dequantize_slot(physical_idx, length)
        if state == COLD_STATE:
            shape = (1, self.kv_heads, length, self.head_dim)
            return (torch.zeros(shape, device=self.device, dtype=torch.float16),
                    torch.zeros(shape, device=self.device, dtype=torch.float16))
        raise ValueError(f"Unsupported block state: {state}")

    def sync_gpu_block_tables(self, layer_idx: int, physical_indices, states) -> None:
        """tierkv_policy.py:450-477."""
        if not self.is_allocated():
            return
        self.full_table_sync_count += 1
        layer_idx = int(layer_idx)
        if layer_idx < 0 or layer_idx >= self.num_layers:
            raise ValueError("layer_idx is out of range.")
        if len(physical_indices) > self.max_blocks_per_layer:
            raise RuntimeError(
                f"Layer {layer_idx} has {len(physical_indices)} blocks, exceeding max_blocks_per_layer="
                f"{self.max_blocks_per_layer}."
            )
        if len(physical_indices) != len(states):
            raise ValueError("Block table and state table lengths must match.")
        for p in physical_indices:
            if not (0 <= int(p) < self._lengths.host.size):
                raise IndexError("index out of range in self")
        self._tables.fill_row(self._T_TABLE, layer_idx, -1)
        self._tables.fill_row(self._T_STATE, layer_idx, COLD_STATE)
        self._tables.fill_row(self._T_LEN, layer_idx, 0)
        for logical_idx, (physical_idx, state) in enumerate(zip(physical_indices, states)):
            self._tables.set(self._T_TABLE, layer_idx, logical_idx, int(physical_idx))
            self._tables.set(self._T_STATE, layer_idx, logical_idx, int(state))
            self._tables.set(self._T_LEN, layer_idx, logical_idx, int(self._lengths.host[int(physical_idx)]))
            self.physical_locations[int(physical_idx)] = (layer_idx, int(logical_idx))

    def get_layer_table(self, layer_idx: int):
        if not self.is_allocated():
            raise RuntimeError("TieredKVTensorPool has not been allocated yet.")
        return self.block_tables[int(layer_idx)], self.block_states[int(layer_idx)]

    def get_layer_lengths(self, layer_idx: int):
        if not self.is_allocated():
            raise RuntimeError("TieredKVTensorPool has not been allocated yet.")
        return self.logical_block_lengths[int(layer_idx)]

    def collect_memory_metrics(self, layer_states: dict) -> dict:
        """tierkv_policy.py:489-654, from the host copies of the tables (no
        device synchronisation)."""
        metrics = _zero_metrics()
        metrics.update({
            "physical_hot_pool_mb": 0.0, "physical_warm_pool_mb": 0.0, "physical_warm_meta_mb": 0.0,
            "physical_total_kv_mb": 0.0, "physical_compression_x": 0.0,
            "hot_slots_used": 0, "hot_slots_capacity": int(self.allocated_pool_blocks),
            "warm_slots_used": 0, "warm_slots_capacity": int(self.allocated_pool_blocks),
            "active_pool_blocks": 0, "allocated_pool_blocks": int(self.allocated_pool_blocks),
            "pool_blocks": int(self.pool_blocks), "pool_utilization": 0.0,
            "capacity_utilization": float(self.allocated_pool_blocks) / max(float(self.pool_blocks), 1.0),
        })
        if not self.is_allocated() or self.kv_heads is None or self.head_dim is None:
            return metrics
        counts = {HOT_STATE: [0, 0], WARM_STATE: [0, 0], COLD_STATE: [0, 0]}
        active_pool_blocks = 0
        for layer_idx in range(self.num_layers):
            layer_state = layer_states.get(layer_idx)
            num_blocks = int(layer_state.num_blocks) if layer_state is not None else 0
            if num_blocks <= 0:
                continue
            table = self._tables.row(self._T_TABLE, layer_idx)[:num_blocks]
            states = self._tables.row(self._T_STATE, layer_idx)[:num_blocks]
            valid = table >= 0
            if not valid.any():
                continue
            lengths = np.maximum(self._lengths.host[table[valid]], 0).astype(np.int64)
            for s in (HOT_STATE, WARM_STATE, COLD_STATE):
                mask = states[valid] == s
                counts[s][0] += int(mask.sum())
                counts[s][1] += int(lengths[mask].sum())
            active_pool_blocks += int(valid.sum())
        lm = _logical_metrics(int(self.kv_heads), int(self.head_dim), counts[HOT_STATE][1],
                              counts[WARM_STATE][1], counts[COLD_STATE][1], self._warm_token_meta_bytes())
        hot_mb = self._tensor_mb(self.hot_k_pool) + self._tensor_mb(self.hot_v_pool)
        warm_mb = self._tensor_mb(self.warm_k_pool) + self._tensor_mb(self.warm_v_pool)
        meta_mb = sum(self._tensor_mb(t) for t in (self.k_scale, self.k_zero, self.v_scale, self.v_zero))
        total_mb = hot_mb + warm_mb + meta_mb
        dense_mb = lm["logical_dense_equivalent_mb"]
        metrics.update({
            "hot_blocks": counts[HOT_STATE][0], "warm_blocks": counts[WARM_STATE][0],
            "cold_blocks": counts[COLD_STATE][0], "hot_tokens": counts[HOT_STATE][1],
            "warm_tokens": counts[WARM_STATE][1], "cold_tokens": counts[COLD_STATE][1],
            "active_tokens": lm["active_tokens"],
            "logical_hot_mb": lm["logical_hot_mb"], "logical_warm_mb": lm["logical_warm_mb"],
            "logical_warm_meta_mb": lm["logical_warm_meta_mb"],
            "logical_cold_evicted_mb": lm["logical_cold_evicted_mb"],
            "logical_dense_equivalent_mb": dense_mb, "logical_resident_mb": lm["logical_resident_mb"],
            "logical_compression_ratio": lm["_resident_b"] / lm["_dense_b"] if lm["_dense_b"] > 0 else 0.0,
            "logical_compression_x": lm["_dense_b"] / lm["_resident_b"] if lm["_resident_b"] > 0 else 0.0,
            "active_pool_blocks": active_pool_blocks,
            "pool_utilization": active_pool_blocks / max(float(self.allocated_pool_blocks), 1.0),
            "physical_hot_pool_mb": hot_mb, "physical_warm_pool_mb": warm_mb,
            "physical_warm_meta_mb": meta_mb, "physical_total_kv_mb": total_mb,
            "physical_compression_x": dense_mb / max(total_mb, 1e-12) if dense_mb > 0 else 0.0,
            "hot_slots_used": counts[HOT_STATE][0], "warm_slots_used": counts[WARM_STATE][0],
        })
        return metrics

    def clear(self) -> None:
        """tierkv_policy.py:662-674 (pool contents are left as they are)."""
        self._launch_queue()
        if self.is_allocated():
            self._lengths.zero()
            self._tables.reset()
        self.physical_states.clear()
        self.physical_locations.clear()
        self.hot_storage.clear()
        self.warm_storage.clear()
        self.cold_storage.clear()
        self.full_table_sync_count = 0

    def release(self) -> None:
        self._launch_queue()
        self.hot_k_pool = None
        self.hot_v_pool = None
        self.warm_k_pool = None
        self.warm_v_pool = None
        self.k_scale = None
        self.k_zero = None
        self.v_scale = None
        self.v_zero = None
        self._lengths = None
        self._tables = None
        self.device = None
        self.kv_heads = None
        self.head_dim = None
        self.allocated_pool_blocks = 0
        self.physical_states.clear()
        self.physical_locations.clear()
        self.hot_storage.clear()
        self.warm_storage.clear()
        self.cold_storage.clear()
        self.full_table_sync_count = 0


# ---------------------------------------------------------------------------
# Compact pool (tierkv_policy.py:701-1365): separate HOT and WARM slot pools,
# tables hold the state-specific slot (-1 for COLD).
# ---------------------------------------------------------------------------

class CompactTieredKVTensorPool(_QueuedStorage):
    _T_PHYS, _T_SLOT, _T_STATE, _T_LEN = 0, 1, 2, 3

    def __init__(
        self,
        num_layers: int = 1,
        block_size: int = 16,
        max_seq_len: int = 2048,
        max_blocks_per_layer: int | None = None,
        pool_blocks: int | None = None,
        pool_chunk_blocks: int = 128,
        max_hot_slots: int | None = None,
        max_warm_slots: int | None = None,
        hot_chunk_slots: int | None = None,
        warm_chunk_slots: int | None = None,
        *,
        warm_format: str = "ref_u8",
    ):
        if num_layers <= 0:
            raise ValueError("num_layers must be positive.")
        if block_size <= 0:
            raise ValueError("block_size must be positive.")
        if max_seq_len <= 0:
            raise ValueError("max_seq_len must be positive.")

        self.num_layers = int(num_layers)
        self.block_size = int(block_size)
        self.max_seq_len = int(max_seq_len)
        self.max_blocks_per_layer = int(max_blocks_per_layer or _ceil_div(max_seq_len, block_size))
        self.pool_blocks = int(pool_blocks or self.num_layers * self.max_blocks_per_layer)
        self.pool_chunk_blocks = int(pool_chunk_blocks)
        self.max_hot_slots = int(max_hot_slots if max_hot_slots is not None else self.pool_blocks)
        self.max_warm_slots = int(max_warm_slots if max_warm_slots is not None else self.pool_blocks)
        self.hot_chunk_slots = int(hot_chunk_slots or self.pool_chunk_blocks)
        self.warm_chunk_slots = int(warm_chunk_slots or self.pool_chunk_blocks)
        if self.max_hot_slots < 0 or self.max_warm_slots < 0:
            raise ValueError("max_hot_slots and max_warm_slots must be non-negative.")
        self.warm_format = self._check_format(warm_format)

        self.device = None
        self.dtype = torch.float16
        self.kv_heads = None
        self.head_dim = None
        self.allocated_pool_blocks = 0
        self.allocated_hot_slots = 0
        self.allocated_warm_slots = 0

        self.hot_k_pool = None
        self.hot_v_pool = None
        self.warm_k_pool = None
        self.warm_v_pool = None
        self.k_scale = None
        self.k_zero = None
        self.v_scale = None
        self.v_zero = None
        self._tables: _Tables | None = None
        self.full_table_sync_count = 0

        self.physical_states: dict[int, int] = {}
        self.physical_locations: dict[int, tuple[int, int]] = {}
        self.physical_lengths: dict[int, int] = {}
        self.physical_slots: dict[int, int] = {}
        self.hot_free_slots: list[int] = []
        self.warm_free_slots: list[int] = []
        self.hot_storage = set()
        self.warm_storage = set()
        self.cold_storage = set()
        self._init_queue()

    @property
    def physical_block_tables(self):
        return None if self._tables is None else self._tables.view(self._T_PHYS)

    @property
    def block_slot_indices(self):
        return None if self._tables is None else self._tables.view(self._T_SLOT)

    @property
    def block_tables(self):
        return self.block_slot_indices

    @property
    def block_states(self):
        return None if self._tables is None else self._tables.view(self._T_STATE)

    @property
    def block_lengths(self):
        return None if self._tables is None else self._tables.view(self._T_LEN)

    def is_allocated(self) -> bool:
        return self._tables is not None

    def _check_physical_idx(self, physical_idx: int) -> int:
        physical_idx = int(physical_idx)
        if physical_idx < 0 or physical_idx >= self.pool_blocks:
            raise RuntimeError(
                f"Physical block {physical_idx} is outside tensor-pool metadata capacity {self.pool_blocks}."
            )
        return physical_idx

    def _ensure_metadata(self, key_states: torch.Tensor) -> None:
        if key_states.ndim != 4 or key_states.shape[0] != 1:
            raise ValueError("KV tensors must have shape [1, kv_heads, tokens, head_dim].")
        device = key_states.device
        kv_heads = int(key_states.shape[1])
        head_dim = int(key_states.shape[-1])
        if self.is_allocated():
            if device != self.device or kv_heads != self.kv_heads or head_dim != self.head_dim:
                raise ValueError("KV tensor geometry changed after tensor-pool allocation.")
            return
        self.device = device
        self.kv_heads = kv_heads
        self.head_dim = head_dim
        self._tables = _Tables((-1, -1, COLD_STATE, 0), self.num_layers, self.max_blocks_per_layer, device)

    def _new_kv_pool(self, capacity: int, dtype):
        return torch.zeros((capacity, self.kv_heads, self.block_size, self.head_dim), device=self.device,
                           dtype=dtype)

    def _ensure_decode_placeholders(self) -> None:
        """One-slot pools so the decode kernel gets valid pointers before the
        first HOT / WARM block exists (tierkv_policy.py:814-826)."""
        if not self.is_allocated():
            return
        if self.hot_k_pool is None:
            self.hot_k_pool = self._new_kv_pool(1, torch.float16)
            self.hot_v_pool = self._new_kv_pool(1, torch.float16)
        if self.warm_k_pool is None:
            self.warm_k_pool = self._new_kv_pool(1, self._warm_dtype())
            self.warm_v_pool = self._new_kv_pool(1, self._warm_dtype())
            self.k_scale = self._new_scale(1, 1)
            self.k_zero = self._new_zero_point(1)
            self.v_scale = self._new_scale(1, 1)
            self.v_zero = self._new_zero_point(1)

    def _grow_hot_slots(self) -> None:
        """tierkv_policy.py:849-869."""
        if self.allocated_hot_slots >= self.max_hot_slots:
            raise RuntimeError("No HOT slots available in compact TierKV pool.")
        self._launch_queue()
        old = self.allocated_hot_slots
        new = min(self.max_hot_slots, old + max(1, self.hot_chunk_slots))
        self.hot_k_pool = self._grow_copy(self.hot_k_pool, self._new_kv_pool(new, torch.float16), old)
        self.hot_v_pool = self._grow_copy(self.hot_v_pool, self._new_kv_pool(new, torch.float16), old)
        self.hot_free_slots.extend(range(new - 1, old - 1, -1))
        self.allocated_hot_slots = new
        self.allocated_pool_blocks = max(self.allocated_hot_slots, self.allocated_warm_slots)

    def _grow_warm_slots(self) -> None:
        """tierkv_policy.py:871-895."""
        if self.allocated_warm_slots >= self.max_warm_slots:
            raise RuntimeError("No WARM slots available in compact TierKV pool.")
        self._launch_queue()
        old = self.allocated_warm_slots
        new = min(self.max_warm_slots, old + max(1, self.warm_chunk_slots))
        self.warm_k_pool = self._grow_copy(self.warm_k_pool, self._new_kv_pool(new, self._warm_dtype()), old)
        self.warm_v_pool = self._grow_copy(self.warm_v_pool, self._new_kv_pool(new, self._warm_dtype()), old)
        self.k_scale = self._grow_copy(self.k_scale, self._new_scale(new, 1), old)
        self.k_zero = self._grow_copy(self.k_zero, self._new_zero_point(new), old)
        self.v_scale = self._grow_copy(self.v_scale, self._new_scale(new, 1), old)
        self.v_zero = self._grow_copy(self.v_zero, self._new_zero_point(new), old)
        self.warm_free_slots.extend(range(new - 1, old - 1, -1))
        self.allocated_warm_slots = new
        self.allocated_pool_blocks = max(self.allocated_hot_slots, self.allocated_warm_slots)

    def _alloc_hot_slot(self) -> int:
        if not self.hot_free_slots:
            self._grow_hot_slots()
        return int(self.hot_free_slots.pop())

    def _alloc_warm_slot(self) -> int:
        if not self.warm_free_slots:
            self._grow_warm_slots()
        return int(self.warm_free_slots.pop())

    def _free_hot_slot(self, slot_idx: int) -> None:
        slot_idx = int(slot_idx)
        if slot_idx >= 0:
            self.hot_free_slots.append(slot_idx)

    def _free_warm_slot(self, slot_idx: int) -> None:
        slot_idx = int(slot_idx)
        if slot_idx >= 0:
            self.warm_free_slots.append(slot_idx)

    def _set_metadata(self, physical_idx: int, state: int, slot_idx: int, length: int) -> None:
        """tierkv_policy.py:917-926."""
        self.physical_states[int(physical_idx)] = int(state)
        self.physical_slots[int(physical_idx)] = int(slot_idx)
        self.physical_lengths[int(physical_idx)] = int(length)
        location = self.physical_locations.get(int(physical_idx))
        if location is not None and self.is_allocated():
            layer_idx, logical_idx = location
            self._tables.set(self._T_STATE, layer_idx, logical_idx, int(state))
            self._tables.set(self._T_SLOT, layer_idx, logical_idx, int(slot_idx))
            self._tables.set(self._T_LEN, layer_idx, logical_idx, int(length))

    def get_physical_state(self, physical_idx: int) -> int | None:
        return self.physical_states.get(int(physical_idx))

    def get_block_length(self, physical_idx: int) -> int:
        return int(self.physical_lengths.get(int(physical_idx), 0))

    def _write_hot_range(self, physical_idx, start, src_k, src_v, tok0, tokens) -> None:
        """write_hot_tokens (934-967) for tokens [tok0, tok0 + tokens) of a whole source."""
        self._ensure_metadata(src_k)
        start, tokens = int(start), int(tokens)
        if start < 0 or start + tokens > self.block_size:
            raise ValueError("KV write exceeds the physical block capacity.")
        current_state = self.get_physical_state(physical_idx)
        if current_state == COLD_STATE:
            raise KeyError(f"Physical block {physical_idx} is COLD and cannot be promoted.")
        if current_state == WARM_STATE:
            self.promote_to_hot(physical_idx)
        slot_idx = self.physical_slots.get(physical_idx)
        if slot_idx is None or current_state is None:
            slot_idx = self._alloc_hot_slot()
        self._queue_write(src_k, src_v, tok0, tokens, slot_idx, start)
        self.hot_storage.add(physical_idx)
        self.warm_storage.discard(physical_idx)
        self.cold_storage.discard(physical_idx)
        self._set_metadata(physical_idx, HOT_STATE, slot_idx, start + tokens)

    def write_hot_tokens(self, physical_idx: int, start: int, key_states: torch.Tensor,
                         value_states: torch.Tensor) -> None:
        physical_idx = self._check_physical_idx(physical_idx)
        key_states, value_states = self._coerce_kv(key_states, value_states)
        with self._batch():
            self._write_hot_range(physical_idx, start, key_states, value_states, 0, key_states.shape[-2])

    def _write_warm_range(self, physical_idx, src_k, src_v, tok0, length) -> None:
        """write_warm_block (969-1002) for tokens [tok0, tok0 + length) of a whole source."""
        self._ensure_metadata(src_k)
        current_state = self.get_physical_state(physical_idx)
        if current_state == HOT_STATE:
            self._free_hot_slot(self.physical_slots.get(physical_idx, -1))
        elif current_state == WARM_STATE:
            self._free_warm_slot(self.physical_slots.get(physical_idx, -1))
        elif current_state == COLD_STATE:
            raise KeyError(f"Physical block {physical_idx} is COLD and cannot be promoted.")
        slot_idx = self._alloc_warm_slot()
        self._queue_stage(src_k, src_v, tok0, length, slot_idx)
        self.hot_storage.discard(physical_idx)
        self.warm_storage.add(physical_idx)
        self.cold_storage.discard(physical_idx)
        self._set_metadata(physical_idx, WARM_STATE, slot_idx, int(length))

    def write_warm_block(self, physical_idx, k_tensor, v_tensor) -> None:
        physical_idx = self._check_physical_idx(physical_idx)
        k_tensor, v_tensor = self._coerce_kv(k_tensor, v_tensor)
        with self._batch():
            self._write_warm_range(physical_idx, k_tensor, v_tensor, 0, k_tensor.shape[-2])

    def register_cold_block(self, physical_idx, length: int) -> None:
        """tierkv_policy.py:1004-1014."""
        physical_idx = self._check_physical_idx(physical_idx)
        state = self.get_physical_state(physical_idx)
        if state == HOT_STATE:
            self._free_hot_slot(self.physical_slots.get(physical_idx, -1))
        elif state == WARM_STATE:
            self._free_warm_slot(self.physical_slots.get(physical_idx, -1))
        self.hot_storage.discard(physical_idx)
        self.warm_storage.discard(physical_idx)
        self.cold_storage.add(physical_idx)
        self._set_metadata(physical_idx, COLD_STATE, -1, int(length))

    def store_hot_block(self, physical_idx, k_tensor, v_tensor) -> None:
        self.write_hot_tokens(int(physical_idx), 0, k_tensor, v_tensor)

    def set_block_entry(self, layer_idx: int, logical_idx: int, physical_idx: int, state: int) -> None:
        """tierkv_policy.py:1019-1035."""
        if not self.is_allocated():
            raise RuntimeError("CompactTieredKVTensorPool has not been allocated yet.")
        layer_idx = int(layer_idx)
        logical_idx = int(logical_idx)
        physical_idx = self._check_physical_idx(physical_idx)
        if layer_idx < 0 or layer_idx >= self.num_layers:
            raise ValueError("layer_idx is out of range.")
        if logical_idx < 0 or logical_idx >= self.max_blocks_per_layer:
            raise RuntimeError(
                f"Logical block {logical_idx} exceeds max_blocks_per_layer={self.max_blocks_per_layer}."
            )
        self.physical_locations[physical_idx] = (layer_idx, logical_idx)
        self._tables.set(self._T_PHYS, layer_idx, logical_idx, physical_idx)
        self._tables.set(self._T_STATE, layer_idx, logical_idx, int(state))
        self._tables.set(self._T_SLOT, layer_idx, logical_idx, int(self.physical_slots.get(physical_idx, -1)))
        self._tables.set(self._T_LEN, layer_idx, logical_idx, int(self.physical_lengths.get(physical_idx, 0)))

    def set_block_state(self, layer_idx: int, logical_idx: int, state: int) -> None:
        if not self.is_allocated():
            raise RuntimeError("CompactTieredKVTensorPool has not been allocated yet.")
        self._tables.set(self._T_STATE, layer_idx, logical_idx, int(state))

    def demote_to_warm(self, physical_idx) -> None:
        """tierkv_policy.py:1042-1068."""
        physical_idx = self._check_physical_idx(physical_idx)
        state = self.get_physical_state(physical_idx)
        if state == WARM_STATE:
            return
        if state == COLD_STATE:
            raise KeyError(f"Physical block {physical_idx} is not eligible for WARM demotion from COLD storage.")
        if state != HOT_STATE:
            raise KeyError(f"Physical block {physical_idx} is not present in HOT storage.")
        length = self.get_block_length(physical_idx)
        hot_slot = self.physical_slots[physical_idx]
        warm_slot = self._alloc_warm_slot()
        self._queue_demote(hot_slot, warm_slot, length)
        self._free_hot_slot(hot_slot)
        self.hot_storage.discard(physical_idx)
        self.warm_storage.add(physical_idx)
        self.cold_storage.discard(physical_idx)
        self._set_metadata(physical_idx, WARM_STATE, warm_slot, length)

    def demote_to_cold(self, physical_idx) -> None:
        """tierkv_policy.py:1070-1085."""
        physical_idx = self._check_physical_idx(physical_idx)
        state = self.get_physical_state(physical_idx)
        if state == COLD_STATE:
            return
        if state == HOT_STATE:
            self._free_hot_slot(self.physical_slots.get(physical_idx, -1))
        elif state == WARM_STATE:
            self._free_warm_slot(self.physical_slots.get(physical_idx, -1))
        elif state is None:
            raise KeyError(f"Physical block {physical_idx} is not present in HOT or WARM storage.")
        length = self.get_block_length(physical_idx)
        self.hot_storage.discard(physical_idx)
        self.warm_storage.discard(physical_idx)
        self.cold_storage.add(physical_idx)
        self._set_metadata(physical_idx, COLD_STATE, -1, length)

    def promote_to_hot(self, physical_idx) -> None:
        """tierkv_policy.py:1087-1115."""
        physical_idx = self._check_physical_idx(physical_idx)
        state = self.get_physical_state(physical_idx)
        if state == HOT_STATE:
            return
        if state == COLD_STATE:
            raise KeyError(f"Physical block {physical_idx} is not eligible for HOT promotion from COLD storage.")
        if state != WARM_STATE:
            raise KeyError(f"Physical block {physical_idx} is not present in WARM storage.")
        length = self.get_block_length(physical_idx)
        warm_slot = self.physical_slots[physical_idx]
        hot_slot = self._alloc_hot_slot()
        self._queue_promote(warm_slot, hot_slot, length)
        self._free_warm_slot(warm_slot)
        self.hot_storage.add(physical_idx)
        self.warm_storage.discard(physical_idx)
        self.cold_storage.discard(physical_idx)
        self._set_metadata(physical_idx, HOT_STATE, hot_slot, length)

    def get_dequantized_block(self, physical_idx, state):
        """tierkv_policy.py:1117-1162."""
        physical_idx = self._check_physical_idx(physical_idx)
        if not self.is_allocated():
            raise KeyError(f"Physical block {physical_idx} is not present in compact tensor-pool storage.")
        length = self.get_block_length(physical_idx)
        actual_state = self.get_physical_state(physical_idx)
        if state == HOT_STATE:
            if actual_state == WARM_STATE:
                self.promote_to_hot(physical_idx)
                actual_state = HOT_STATE
            if actual_state == COLD_STATE:
                raise KeyError(f"Physical block {physical_idx} is marked HOT but only exists in COLD storage.")
            self._launch_queue()
            slot_idx = self.physical_slots[physical_idx]
            return (self.hot_k_pool[slot_idx: slot_idx + 1, :, :length, :].contiguous(),
                    self.hot_v_pool[slot_idx: slot_idx + 1, :, :length, :].contiguous())
        if state == WARM_STATE:
            if actual_state == COLD_STATE:
                raise KeyError(f"Physical block {physical_idx} is marked WARM but only exists in COLD storage.")
            self._launch_queue()
            slot_idx = self.physical_slots[physical_idx]
            if actual_state == HOT_STATE:
                return (self.hot_k_pool[slot_idx: slot_idx + 1, :, :length, :].contiguous(),
                        self.hot_v_pool[slot_idx: slot_idx + 1, :, :length, :].contiguous())
            return self._dequantize_slot(slot_idx, length)
        if state == COLD_STATE:
            shape = (1, self.kv_heads, length, self.head_dim)
            return (torch.zeros(shape, device=self.device, dtype=torch.float16),
                    torch.zeros(shape, device=self.device, dtype=torch.float16))
        raise ValueError(f"Unsupported block state: {state}")

    def sync_gpu_block_tables(self, layer_idx: int, physical_indices, states) -> None:
        """tierkv_policy.py:1164-1174."""
        if not self.is_allocated():
            return
        self.full_table_sync_count += 1
        layer_idx = int(layer_idx)
        for k, fill in ((self._T_PHYS, -1), (self._T_SLOT, -1), (self._T_STATE, COLD_STATE), (self._T_LEN, 0)):
            self._tables.fill_row(k, layer_idx, fill)
        for logical_idx, (physical_idx, state) in enumerate(zip(physical_indices, states)):
            self.set_block_entry(layer_idx, logical_idx, int(physical_idx), int(state))

    def get_layer_table(self, layer_idx: int):
        if not self.is_allocated():
            raise RuntimeError("CompactTieredKVTensorPool has not been allocated yet.")
        self._ensure_decode_placeholders()
        return self.block_slot_indices[int(layer_idx)], self.block_states[int(layer_idx)]

    def get_layer_lengths(self, layer_idx: int):
        if not self.is_allocated():
            raise RuntimeError("CompactTieredKVTensorPool has not been allocated yet.")
        return self.block_lengths[int(layer_idx)]

    def collect_memory_metrics(self, layer_states: dict) -> dict:
        """tierkv_policy.py:1193-1317, from the host copies of the tables."""
        hot_mb = self._tensor_mb(self.hot_k_pool) + self._tensor_mb(self.hot_v_pool)
        warm_mb = self._tensor_mb(self.warm_k_pool) + self._tensor_mb(self.warm_v_pool)
        meta_mb = sum(self._tensor_mb(t) for t in (self.k_scale, self.k_zero, self.v_scale, self.v_zero))
        metrics = _zero_metrics()
        metrics.update({
            "active_pool_blocks": 0, "allocated_pool_blocks": int(self.allocated_pool_blocks),
            "pool_blocks": int(self.pool_blocks), "pool_utilization": 0.0, "capacity_utilization": 0.0,
            "physical_hot_pool_mb": hot_mb, "physical_warm_pool_mb": warm_mb, "physical_warm_meta_mb": meta_mb,
            "physical_total_kv_mb": hot_mb + warm_mb + meta_mb, "physical_compression_x": 0.0,
            "hot_slots_used": len(self.hot_storage), "hot_slots_capacity": int(self.allocated_hot_slots),
            "warm_slots_used": len(self.warm_storage), "warm_slots_capacity": int(self.allocated_warm_slots),
        })
        if not self.is_allocated() or self.kv_heads is None or self.head_dim is None:
            return metrics
        counts = {HOT_STATE: [0, 0], WARM_STATE: [0, 0], COLD_STATE: [0, 0]}
        for layer_idx in range(self.num_layers):
            layer_state = layer_states.get(layer_idx)
            num_blocks = int(layer_state.num_blocks) if layer_state is not None else 0
            if num_blocks <= 0:
                continue
            states = self._tables.row(self._T_STATE, layer_idx)[:num_blocks]
            lengths = self._tables.row(self._T_LEN, layer_idx)[:num_blocks].astype(np.int64)
            for s in (HOT_STATE, WARM_STATE, COLD_STATE):
                mask = states == s
                counts[s][0] += int(mask.sum())
                counts[s][1] += int(lengths[mask].sum())
        lm = _logical_metrics(int(self.kv_heads), int(self.head_dim), counts[HOT_STATE][1],
                              counts[WARM_STATE][1], counts[COLD_STATE][1], self._warm_token_meta_bytes())
        dense_mb = lm["logical_dense_equivalent_mb"]
        resident_mb = lm["logical_resident_mb"]
        resident_blocks = counts[HOT_STATE][0] + counts[WARM_STATE][0]
        allocated = self.allocated_hot_slots + self.allocated_warm_slots
        total_mb = hot_mb + warm_mb + meta_mb
        metrics.update({
            "hot_blocks": counts[HOT_STATE][0], "warm_blocks": counts[WARM_STATE][0],
            "cold_blocks": counts[COLD_STATE][0], "hot_tokens": counts[HOT_STATE][1],
            "warm_tokens": counts[WARM_STATE][1], "cold_tokens": counts[COLD_STATE][1],
            "active_tokens": lm["active_tokens"],
            "logical_hot_mb": lm["logical_hot_mb"], "logical_warm_mb": lm["logical_warm_mb"],
            "logical_warm_meta_mb": lm["logical_warm_meta_mb"],
            "logical_cold_evicted_mb": lm["logical_cold_evicted_mb"],
            "logical_dense_equivalent_mb": dense_mb, "logical_resident_mb": resident_mb,
            "logical_compression_ratio": resident_mb / dense_mb if dense_mb > 0 else 0.0,
            "logical_compression_x": dense_mb / resident_mb if resident_mb > 0 else 0.0,
            "active_pool_blocks": resident_blocks,
            "allocated_pool_blocks": int(allocated),
            "pool_blocks": int(self.max_hot_slots + self.max_warm_slots),
            "pool_utilization": resident_blocks / max(float(allocated), 1.0),
            "capacity_utilization": allocated / max(float(self.max_hot_slots + self.max_warm_slots), 1.0),
            "physical_compression_x": dense_mb / total_mb if total_mb > 0 else 0.0,
        })
        return metrics

    def clear(self) -> None:
        """tierkv_policy.py:1319-1334 (pool contents are left as they are)."""
        self._launch_queue()
        if self.is_allocated():
            self._tables.reset()
        self.physical_states.clear()
        self.physical_locations.clear()
        self.physical_lengths.clear()
        self.physical_slots.clear()
        self.hot_storage.clear()
        self.warm_storage.clear()
        self.cold_storage.clear()
        self.hot_free_slots = list(range(self.allocated_hot_slots - 1, -1, -1))
        self.warm_free_slots = list(range(self.allocated_warm_slots - 1, -1, -1))
        self.full_table_sync_count = 0

    def release(self) -> None:
        self._launch_queue()
        self.hot_k_pool = None
        self.hot_v_pool = None
        self.warm_k_pool = None
        self.warm_v_pool = None
        self.k_scale = None
        self.k_zero = None
        self.v_scale = None
        self.v_zero = None
        self._tables = None
        self.device = None
        self.kv_heads = None
        self.head_dim = None
        self.allocated_pool_blocks = 0
        self.allocated_hot_slots = 0
        self.allocated_warm_slots = 0
        self.physical_states.clear()
        self.physical_locations.clear()
        self.physical_lengths.clear()
        self.physical_slots.clear()
        self.hot_free_slots.clear()
        self.warm_free_slots.clear()
        self.hot_storage.clear()
        self.warm_storage.clear()
        self.cold_storage.clear()
        self.full_table_sync_count = 0


# The reference keeps the old public name for its tests (tierkv_policy.py:1368-1369).
PhysicalKVPool = TieredKVTensorPool


# ---------------------------------------------------------------------------
# Policy engine (tierkv_policy.py:1372-1478).
# ---------------------------------------------------------------------------

def _score_device(block_scores: torch.Tensor) -> torch.device:
    if isinstance(block_scores, torch.Tensor) and block_scores.is_cuda:
        return block_scores.device
    return torch.device("cuda", torch.cuda.current_device())


def _labels(block_scores, current_states, hot_budget, warm_budget, mode, demoted_state=WARM_STATE) -> list[int]:
    """Stable-rank labels for one sequence from the label kernel; one
    device-to-host copy."""
    device = _score_device(block_scores)
    scores = block_scores.to(device=device, dtype=torch.float32).contiguous()
    cur = stage_i32(np.asarray(current_states, np.int32), device)
    out = torch.empty_like(cur)
    lib = _lib.lib()
    rc = lib.tierkv_tier_labels(_lib.ptr(scores), _lib.ptr(cur), _lib.ptr(out), int(cur.numel()), 1,
                                int(scores.numel()), int(hot_budget), int(warm_budget), LABEL_MODES[mode],
                                int(demoted_state), _lib.stream_of(device))
    _lib.check(rc, "tierkv_tier_labels")
    return out.cpu().tolist()


class TierKVPolicyEngine:
    def __init__(self, block_size: int, block_manager):
        if block_size <= 0:
            raise ValueError("block_size must be positive.")
        self.block_size = block_size
        self.block_manager = block_manager

    def compute_block_scores(self, attn_weights: torch.Tensor) -> torch.Tensor:
        """Mean attention per block over (batch, heads, queries) and the block's
        tokens (tierkv_policy.py:1380-1389), in the block-mass kernel; fp32
        accumulation, result in the weights' dtype."""
        if attn_weights.ndim != 4:
            raise ValueError("attn_weights must have shape [batch, num_heads, query_seq_len, past_seq_len].")
        if attn_weights.shape[-1] == 0:
            raise ValueError("attn_weights past_seq_len must be positive.")
        _lib.require_gpu_tensor(attn_weights, "attn_weights")
        lib = _lib.lib()
        tokens = int(attn_weights.shape[-1])
        rows = attn_weights.numel() // tokens
        bs = int(self.block_size)
        nblk = _ceil_div(tokens, bs)
        probs = torch.zeros((1, rows, nblk * bs), dtype=torch.float32, device=attn_weights.device)
        probs[0, :, :tokens].copy_(attn_weights.reshape(rows, tokens))
        lengths = np.full(nblk, bs, np.int32)
        lengths[-1] = tokens - bs * (nblk - 1)
        ln = stage_i32(lengths, attn_weights.device)
        out = torch.empty((1, nblk), dtype=torch.float32, device=attn_weights.device)
        rc = lib.tierkv_block_mass_from_probs(_lib.ptr(probs), _lib.ptr(ln), _lib.ptr(out), 1, rows,
                                              nblk * bs, bs, _lib.stream_of(attn_weights.device))
        _lib.check(rc, "tierkv_block_mass_from_probs")
        return out[0].to(attn_weights.dtype)

    def _checked_states(self, seq_id, block_scores):
        physical_indices = self.block_manager.get_physical_indices(seq_id)
        current_states = self.block_manager.get_states(seq_id)
        return physical_indices, current_states

    def _apply(self, seq_id, current_states, desired) -> None:
        for block_idx, (cur, want) in enumerate(zip(current_states, desired)):
            if cur != want:
                self.block_manager.update_block_state(seq_id, block_idx, int(want))

    def enforce_budget(self, seq_id: int, block_scores: torch.Tensor, hot_budget: int,
                       demoted_state: int = WARM_STATE):
        """tierkv_policy.py:1391-1432."""
        physical_indices, current_states = self._checked_states(seq_id, block_scores)
        num_blocks = len(physical_indices)
        if num_blocks == 0:
            return
        if demoted_state not in (WARM_STATE, COLD_STATE):
            raise ValueError("demoted_state must be WARM_STATE or COLD_STATE.")
        if block_scores.ndim != 1:
            raise ValueError("block_scores must be a 1D tensor.")
        if len(block_scores) != num_blocks:
            raise ValueError("block_scores length must match the allocated block count.")
        if len(current_states) != num_blocks:
            raise ValueError("Block state table is inconsistent with physical index table.")
        if num_blocks <= 2:
            self._apply(seq_id, current_states, [HOT_STATE] * num_blocks)
            return
        desired = _labels(block_scores, current_states, hot_budget, 0, "hot_warm", demoted_state)
        self._apply(seq_id, current_states, desired)

    def enforce_tiered_budget(self, seq_id: int, block_scores: torch.Tensor, hot_budget: int, warm_budget: int):
        """tierkv_policy.py:1434-1477."""
        physical_indices, current_states = self._checked_states(seq_id, block_scores)
        num_blocks = len(physical_indices)
        if num_blocks == 0:
            return
        if block_scores.ndim != 1:
            raise ValueError("block_scores must be a 1D tensor.")
        if len(block_scores) != num_blocks:
            raise ValueError("block_scores length must match the allocated block count.")
        if len(current_states) != num_blocks:
            raise ValueError("Block state table is inconsistent with physical index table.")
        if num_blocks <= 2:
            self._apply(seq_id, current_states, [HOT_STATE] * num_blocks)
            return
        desired = _labels(block_scores, current_states, hot_budget, warm_budget, "hot_warm_cold")
        self._apply(seq_id, current_states, desired)


@dataclass
class LayerRuntimeState:
    open_physical_idx: int | None = None
    open_token_count: int = 0
    num_blocks: int = 0


class TieredKVCache(HFCache):
    """The HF cache object of a tiered runtime (tierkv_policy.py:1487-1531):
    it only tracks the committed sequence length; the KV lives in the runtime."""

    is_compileable = False

    def __init__(self, runtime):
        self.runtime = runtime
        self.is_tierkv_cache = True
        self.pending_query_length = 0
        self.committed_seq_len = 0

    def begin_forward(self, query_length: int) -> None:
        self.pending_query_length = int(query_length)
        self.runtime.begin_forward(query_length)

    def finish_forward(self) -> None:
        self.committed_seq_len += self.pending_query_length
        self.pending_query_length = 0
        self.runtime.finish_forward()

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.committed_seq_len

    def get_mask_sizes(self, query_length: int, layer_idx: int = 0) -> tuple[int, int]:
        return self.committed_seq_len + int(query_length), 0

    def get_max_cache_shape(self, layer_idx: int = 0) -> int:
        return -1

    def reset(self) -> None:
        self.pending_query_length = 0
        self.committed_seq_len = 0

    def reorder_cache(self, beam_idx: torch.LongTensor):
        return None

    def crop(self, max_length: int):
        return None

    def batch_repeat_interleave(self, repeats: int):
        return None

    def batch_select_indices(self, indices: torch.Tensor):
        return None

    def __len__(self):
        return self.runtime.num_layers


# ---------------------------------------------------------------------------
# Runtime (tierkv_policy.py:1534-1912).
# ---------------------------------------------------------------------------

class TieredKVRuntime:
    def __init__(
        self,
        block_manager,
        num_layers: int,
        block_size: int,
        hot_budget: int,
        max_seq_len: int = 2048,
        attention_backend: str | None = None,
        policy_interval: int | None = None,
        pool_chunk_blocks: int = 128,
        policy_on_new_block: bool = False,
        score_accumulation_mode: str = "policy_ticks",
        policy_mode: str = "hot_warm",
        warm_budget: int = 32,
        pool_layout: str | None = None,
        *,
        warm_format: str = "ref_u8",
        prefill_scoring: str = "proxy",
    ):
        attention_backend = attention_backend or os.environ.get("TIERKV_ATTENTION_BACKEND", "triton")
        if prefill_scoring not in ("proxy", "attention"):
            raise ValueError('prefill_scoring must be "proxy" or "attention".')
        # Prefill block scores when the model's attention returns no
        # probabilities: "proxy" = the reference's sink + recency scores,
        # "attention" = the prefill block-score kernel (extension).
        self.prefill_scoring = prefill_scoring
        if attention_backend not in ("eager", "triton"):
            raise ValueError('attention_backend must be "eager" or "triton".')
        if policy_interval is None:
            policy_interval = int(os.environ.get("TIERKV_POLICY_INTERVAL", "16"))
        if policy_interval <= 0:
            raise ValueError("policy_interval must be positive.")
        pool_chunk_blocks = int(os.environ.get("TIERKV_POOL_CHUNK_BLOCKS", pool_chunk_blocks))
        if pool_chunk_blocks <= 0:
            raise ValueError("pool_chunk_blocks must be positive.")
        policy_on_new_block = os.environ.get("TIERKV_POLICY_ON_NEW_BLOCK", str(policy_on_new_block)).lower()
        policy_on_new_block = policy_on_new_block in ("1", "true", "yes", "on")
        score_accumulation_mode = os.environ.get("TIERKV_SCORE_ACCUMULATION_MODE", score_accumulation_mode)
        if score_accumulation_mode not in ("policy_ticks", "every_step"):
            raise ValueError('score_accumulation_mode must be "policy_ticks" or "every_step".')
        policy_mode = os.environ.get("TIERKV_POLICY_MODE", policy_mode)
        if policy_mode not in ("hot_only", "hot_warm", "hot_warm_cold"):
            raise ValueError('policy_mode must be "hot_only", "hot_warm", or "hot_warm_cold".')
        warm_budget = int(os.environ.get("TIERKV_WARM_BUDGET", warm_budget))
        if warm_budget < 0:
            raise ValueError("warm_budget must be non-negative.")
        pool_layout = os.environ.get("TIERKV_POOL_LAYOUT", pool_layout or "compact")
        if pool_layout not in ("compact", "dense"):
            raise ValueError('pool_layout must be "compact" or "dense".')

        self.block_manager = block_manager
        self.num_layers = int(num_layers)
        self.block_size = int(block_size)
        self.hot_budget = int(hot_budget)
        self.max_seq_len = int(max_seq_len)
        self.max_blocks_per_layer = _ceil_div(self.max_seq_len, self.block_size)
        self.pool_blocks = self.num_layers * self.max_blocks_per_layer
        self.attention_backend = attention_backend
        self.policy_interval = int(policy_interval)
        self.pool_chunk_blocks = int(pool_chunk_blocks)
        self.policy_on_new_block = bool(policy_on_new_block)
        self.score_accumulation_mode = score_accumulation_mode
        self.policy_mode = policy_mode
        self.warm_budget = int(warm_budget)
        self.pool_layout = pool_layout
        self.demoted_state = WARM_STATE
        self.cold_block_policy = "zero"
        self.tiered_layer_indices = set(range(num_layers))
        if self.pool_layout == "compact":
            hot_slots_per_layer, warm_slots_per_layer = self._compact_slot_capacities()
            self.kv_pool = CompactTieredKVTensorPool(
                num_layers=self.num_layers,
                block_size=self.block_size,
                max_seq_len=self.max_seq_len,
                max_blocks_per_layer=self.max_blocks_per_layer,
                pool_blocks=self.pool_blocks,
                pool_chunk_blocks=self.pool_chunk_blocks,
                max_hot_slots=self.num_layers * hot_slots_per_layer,
                max_warm_slots=self.num_layers * warm_slots_per_layer,
                hot_chunk_slots=max(1, hot_slots_per_layer),
                warm_chunk_slots=max(1, warm_slots_per_layer),
                warm_format=warm_format,
            )
        else:
            self.kv_pool = TieredKVTensorPool(
                num_layers=self.num_layers,
                block_size=self.block_size,
                max_seq_len=self.max_seq_len,
                max_blocks_per_layer=self.max_blocks_per_layer,
                pool_blocks=self.pool_blocks,
                pool_chunk_blocks=self.pool_chunk_blocks,
                warm_format=warm_format,
            )
        self.policy_engine = TierKVPolicyEngine(block_size=block_size, block_manager=block_manager)
        self.layer_states = {layer_idx: LayerRuntimeState() for layer_idx in range(num_layers)}
        self.cache = TieredKVCache(self)
        self.current_query_length = 0
        self.decode_step = 0
        self.policy_tick_this_forward = False
        self.profile_enabled = os.environ.get("TIERKV_PROFILE", "0") == "1"
        self.profile_totals_ms: dict[str, float] = {}
        self.profile_counts: dict[str, int] = {}

    def _compact_slot_capacities(self) -> tuple[int, int]:
        """tierkv_policy.py:1628-1637."""
        if self.policy_mode == "hot_only":
            return self.max_blocks_per_layer, 0
        hot_slack = _ceil_div(self.policy_interval, self.block_size) + 2
        hot_slots = min(self.max_blocks_per_layer, max(2, self.hot_budget) + hot_slack)
        if self.policy_mode == "hot_warm_cold":
            warm_slots = min(self.max_blocks_per_layer, self.warm_budget + 2)
        else:
            warm_slots = self.max_blocks_per_layer
        return max(1, hot_slots), max(0, warm_slots)

    def begin_forward(self, query_length: int) -> None:
        self.current_query_length = int(query_length)
        self.policy_tick_this_forward = False
        if self.current_query_length == 1:
            self.decode_step += 1
            self.policy_tick_this_forward = (self.decode_step % self.policy_interval) == 0

    def finish_forward(self) -> None:
        self.current_query_length = 0
        self.policy_tick_this_forward = False

    def reset(self, release_storage: bool = False) -> None:
        for seq_id in range(self.num_layers):
            self.block_manager.free_sequence(seq_id)
        if release_storage:
            self.kv_pool.release()
        else:
            self.kv_pool.clear()
        self.layer_states = {layer_idx: LayerRuntimeState() for layer_idx in range(self.num_layers)}
        self.decode_step = 0
        self.current_query_length = 0
        self.policy_tick_this_forward = False
        self.profile_totals_ms.clear()
        self.profile_counts.clear()
        self.cache.reset()

    def profile_start(self):
        if not self.profile_enabled or not torch.cuda.is_available():
            return None
        event = torch.cuda.Event(enable_timing=True)
        event.record()
        return event

    def profile_end(self, name: str, start_event) -> None:
        if start_event is None:
            return
        end_event = torch.cuda.Event(enable_timing=True)
        end_event.record()
        end_event.synchronize()
        elapsed = float(start_event.elapsed_time(end_event))
        self.profile_totals_ms[name] = self.profile_totals_ms.get(name, 0.0) + elapsed
        self.profile_counts[name] = self.profile_counts.get(name, 0) + 1

    def profile_summary(self) -> dict[str, tuple[float, int, float]]:
        summary = {}
        for name, total_ms in self.profile_totals_ms.items():
            count = self.profile_counts.get(name, 0)
            summary[name] = (total_ms, count, total_ms / max(count, 1))
        return summary

    def collect_memory_metrics(self) -> dict:
        return self.kv_pool.collect_memory_metrics(self.layer_states)

    def append_tokens(self, layer_idx: int, key_states: torch.Tensor, value_states: torch.Tensor) -> bool:
        return self.append_to_layer(layer_idx, key_states, value_states)

    def _desired_prefill_states(self, num_blocks: int, block_scores: torch.Tensor) -> list[int]:
        """tierkv_policy.py:1695-1720, ranked by the label kernel."""
        if self.policy_mode == "hot_only" or num_blocks <= 2:
            return [HOT_STATE] * int(num_blocks)
        if block_scores.ndim != 1 or len(block_scores) != int(num_blocks):
            raise ValueError("block_scores must be a 1D tensor matching prefill block count.")
        if self.policy_mode == "hot_warm_cold":
            return _labels(block_scores, [HOT_STATE] * int(num_blocks), self.hot_budget, self.warm_budget,
                           "hot_warm_cold")
        return _labels(block_scores, [HOT_STATE] * int(num_blocks), self.hot_budget, 0, "hot_warm",
                       self.demoted_state)

    def append_prefill_with_policy(self, seq_id: int, key_states: torch.Tensor, value_states: torch.Tensor,
                                   block_scores: torch.Tensor) -> None:
        """tierkv_policy.py:1722-1766: every block goes straight to its tier
        (HOT copied, WARM quantized, COLD metadata only); one copy launch and
        one quantize launch for the whole prompt."""
        if key_states.shape[-2] != value_states.shape[-2]:
            raise ValueError("Key and value states must have the same sequence length.")
        layer_state = self.layer_states[seq_id]
        if layer_state.num_blocks != 0 or layer_state.open_physical_idx is not None:
            raise RuntimeError("append_prefill_with_policy expects an empty layer cache.")
        total_tokens = int(key_states.shape[-2])
        num_blocks = _ceil_div(total_tokens, self.block_size)
        if num_blocks > self.max_blocks_per_layer:
            raise RuntimeError(f"Layer {seq_id} exceeded max_blocks_per_layer={self.max_blocks_per_layer}.")
        desired_states = self._desired_prefill_states(num_blocks, block_scores)
        pool = self.kv_pool
        src_k, src_v = pool._source(key_states, value_states)
        with pool._batch():
            for logical_idx, desired_state in enumerate(desired_states):
                physical_idx = self.block_manager.allocate_block(seq_id)
                if desired_state != HOT_STATE:
                    self.block_manager.update_block_state(seq_id, logical_idx, desired_state)
                start = logical_idx * self.block_size
                length = min(start + self.block_size, total_tokens) - start
                physical_idx = pool._check_physical_idx(physical_idx)
                if desired_state == HOT_STATE:
                    pool._write_hot_range(physical_idx, 0, src_k, src_v, start, length)
                elif desired_state == WARM_STATE:
                    pool._write_warm_range(physical_idx, src_k, src_v, start, length)
                elif desired_state == COLD_STATE:
                    if not pool.is_allocated():
                        pool._write_hot_range(physical_idx, 0, src_k, src_v, start, length)
                        pool.demote_to_cold(physical_idx)
                    else:
                        pool.register_cold_block(physical_idx, length)
                else:
                    raise ValueError(f"Unsupported desired state: {desired_state}")
                pool.set_block_entry(seq_id, logical_idx, physical_idx, desired_state)
        layer_state.num_blocks = num_blocks
        layer_state.open_physical_idx = None
        layer_state.open_token_count = 0

    def append_to_layer(self, seq_id: int, key_states: torch.Tensor, value_states: torch.Tensor) -> bool:
        """tierkv_policy.py:1768-1816: fill the open block, then new HOT blocks."""
        if key_states.shape[-2] != value_states.shape[-2]:
            raise ValueError("Key and value states must have the same sequence length.")
        layer_state = self.layer_states[seq_id]
        offset = 0
        total_tokens = int(key_states.shape[-2])
        allocated_new_block = False
        pool = self.kv_pool
        src_k, src_v = pool._source(key_states, value_states)
        with pool._batch():
            while offset < total_tokens:
                new_logical_idx = None
                if layer_state.open_physical_idx is None:
                    layer_state.open_physical_idx = self.block_manager.allocate_block(seq_id)
                    layer_state.open_token_count = 0
                    allocated_new_block = True
                    new_logical_idx = layer_state.num_blocks
                    if new_logical_idx >= self.max_blocks_per_layer:
                        raise RuntimeError(
                            f"Layer {seq_id} exceeded max_blocks_per_layer={self.max_blocks_per_layer}."
                        )
                    pool._check_physical_idx(layer_state.open_physical_idx)
                physical_idx = layer_state.open_physical_idx
                if pool.get_physical_state(physical_idx) == WARM_STATE:
                    pool.promote_to_hot(physical_idx)
                take = min(self.block_size - layer_state.open_token_count, total_tokens - offset)
                pool._write_hot_range(physical_idx, layer_state.open_token_count, src_k, src_v, offset, take)
                if new_logical_idx is not None:
                    pool.set_block_entry(seq_id, new_logical_idx, physical_idx, HOT_STATE)
                    layer_state.num_blocks += 1
                layer_state.open_token_count += take
                offset += take
                if layer_state.open_token_count == self.block_size:
                    layer_state.open_physical_idx = None
                    layer_state.open_token_count = 0
        return allocated_new_block

    def reconstruct_layer(self, seq_id: int, allow_decode_reconstruct: bool = False):
        """tierkv_policy.py:1818-1841."""
        if self.attention_backend == "triton" and self.current_query_length == 1 and not allow_decode_reconstruct:
            raise RuntimeError("Decode reconstruction is disabled for the Triton TierKV hot path.")
        physical_indices = self.block_manager.get_physical_indices(seq_id)
        states = self.block_manager.get_states(seq_id)
        if not physical_indices:
            return None, None, physical_indices, states
        key_blocks, value_blocks = [], []
        for physical_idx, state in zip(physical_indices, states):
            key_block, value_block = self.kv_pool.get_dequantized_block(physical_idx, state)
            key_blocks.append(key_block)
            value_blocks.append(value_block)
        key_states = torch.cat(key_blocks, dim=-2).contiguous()
        value_states = torch.cat(value_blocks, dim=-2).contiguous()
        return key_states, value_states, physical_indices, states

    def sync_gpu_block_tables(self, seq_id: int) -> None:
        physical_indices = self.block_manager.get_physical_indices(seq_id)
        states = self.block_manager.get_states(seq_id)
        self.kv_pool.sync_gpu_block_tables(seq_id, physical_indices, states)
        self.layer_states[seq_id].num_blocks = len(physical_indices)

    def sync_storage_states(self, seq_id: int) -> None:
        """tierkv_policy.py:1849-1867: every migration of the layer in one
        batch (one demote launch, one promote launch, one table push)."""
        physical_indices = self.block_manager.get_physical_indices(seq_id)
        states = self.block_manager.get_states(seq_id)
        pool = self.kv_pool
        with pool._batch():
            for logical_idx, (physical_idx, state) in enumerate(zip(physical_indices, states)):
                current_state = pool.get_physical_state(physical_idx)
                if state == HOT_STATE:
                    if current_state == WARM_STATE:
                        pool.promote_to_hot(physical_idx)
                    elif current_state == COLD_STATE:
                        raise KeyError(f"Physical block {physical_idx} cannot be promoted from COLD to HOT.")
                elif state == COLD_STATE and current_state != COLD_STATE:
                    pool.demote_to_cold(physical_idx)
                elif state == WARM_STATE:
                    if current_state == HOT_STATE:
                        pool.demote_to_warm(physical_idx)
                    elif current_state == COLD_STATE:
                        raise KeyError(f"Physical block {physical_idx} cannot be promoted from COLD to WARM.")
                pool.set_block_state(seq_id, logical_idx, state)

    def get_layer_table(self, seq_id: int):
        block_table, block_states = self.kv_pool.get_layer_table(seq_id)
        num_blocks = self.layer_states[seq_id].num_blocks
        return block_table, block_states, self.kv_pool.get_layer_lengths(seq_id), num_blocks

    def should_run_decode_policy(self, seq_id: int, allocated_new_block: bool) -> bool:
        return (
            seq_id in self.tiered_layer_indices
            and self.policy_mode != "hot_only"
            and self.current_query_length == 1
            and (self.policy_tick_this_forward or (self.policy_on_new_block and allocated_new_block))
        )

    def should_collect_decode_scores(self, seq_id: int, run_policy: bool) -> bool:
        if seq_id not in self.tiered_layer_indices or self.policy_mode == "hot_only":
            return False
        return bool(run_policy or self.score_accumulation_mode == "every_step")

    def enforce_policy(self, seq_id: int, block_scores: torch.Tensor) -> None:
        if self.policy_mode == "hot_only":
            return
        if self.policy_mode == "hot_warm_cold":
            self.policy_engine.enforce_tiered_budget(seq_id, block_scores, self.hot_budget, self.warm_budget)
            return
        self.policy_engine.enforce_budget(seq_id, block_scores, self.hot_budget, demoted_state=self.demoted_state)

    def block_scores_from_probability_sums(self, seq_id: int, score_sums: torch.Tensor) -> torch.Tensor:
        """tierkv_policy.py:1905-1912 in the block-score kernel."""
        num_blocks = self.layer_states[seq_id].num_blocks
        if num_blocks == 0:
            return torch.empty(0, device=score_sums.device, dtype=torch.float32)
        _lib.require_gpu_tensor(score_sums, "score_sums")
        lengths = self.kv_pool.get_layer_lengths(seq_id)
        sums = score_sums.to(torch.float32).contiguous()
        heads, stride = int(sums.shape[0]), int(sums.shape[1])
        out = torch.empty(num_blocks, dtype=torch.float32, device=sums.device)
        rc = _lib.lib().tierkv_block_scores_from_sums(_lib.ptr(sums), stride, _lib.ptr(lengths), int(lengths.numel()),
                                                     _lib.ptr(out), 1, heads, num_blocks, _lib.stream_of(sums.device))
        _lib.check(rc, "tierkv_block_scores_from_sums")
        return out


# ---------------------------------------------------------------------------
# Module-level runtime handle (tierkv_policy.py:1915-2044).
# ---------------------------------------------------------------------------

def initialize_global_tierkv(
    block_manager,
    num_layers,
    block_size=16,
    hot_budget=3,
    max_seq_len=2048,
    attention_backend: str | None = None,
    policy_interval: int | None = None,
    pool_chunk_blocks: int = 128,
    policy_on_new_block: bool = False,
    score_accumulation_mode: str = "policy_ticks",
    policy_mode: str = "hot_warm",
    warm_budget: int = 32,
    pool_layout: str | None = None,
    *,
    warm_format: str = "ref_u8",
) -> TieredKVCache:
    global _GLOBAL_TIERKV_RUNTIME
    if _GLOBAL_TIERKV_RUNTIME is not None:
        _GLOBAL_TIERKV_RUNTIME.reset(release_storage=True)
    _GLOBAL_TIERKV_RUNTIME = create_tierkv_runtime(
        block_manager=block_manager, num_layers=num_layers, block_size=block_size, hot_budget=hot_budget,
        max_seq_len=max_seq_len, attention_backend=attention_backend, policy_interval=policy_interval,
        pool_chunk_blocks=pool_chunk_blocks, policy_on_new_block=policy_on_new_block,
        score_accumulation_mode=score_accumulation_mode, policy_mode=policy_mode, warm_budget=warm_budget,
        pool_layout=pool_layout, warm_format=warm_format,
    )
    return _GLOBAL_TIERKV_RUNTIME.cache


def create_tierkv_runtime(
    block_manager,
    num_layers,
    block_size=16,
    hot_budget=3,
    max_seq_len=2048,
    attention_backend: str | None = None,
    policy_interval: int | None = None,
    pool_chunk_blocks: int = 128,
    policy_on_new_block: bool = False,
    score_accumulation_mode: str = "policy_ticks",
    policy_mode: str = "hot_warm",
    warm_budget: int = 32,
    pool_layout: str | None = None,
    *,
    warm_format: str = "ref_u8",
) -> TieredKVRuntime:
    return TieredKVRuntime(
        block_manager=block_manager, num_layers=num_layers, block_size=block_size, hot_budget=hot_budget,
        max_seq_len=max_seq_len, attention_backend=attention_backend, policy_interval=policy_interval,
        pool_chunk_blocks=pool_chunk_blocks, policy_on_new_block=policy_on_new_block,
        score_accumulation_mode=score_accumulation_mode, policy_mode=policy_mode, warm_budget=warm_budget,
        pool_layout=pool_layout, warm_format=warm_format,
    )


_SUMMED_KEYS = (
    "hot_blocks", "warm_blocks", "cold_blocks", "hot_tokens", "warm_tokens", "cold_tokens", "active_tokens",
    "logical_hot_mb", "logical_warm_mb", "logical_warm_meta_mb", "logical_cold_evicted_mb",
    "logical_dense_equivalent_mb", "logical_resident_mb", "physical_hot_pool_mb", "physical_warm_pool_mb",
    "physical_warm_meta_mb", "physical_total_kv_mb", "active_pool_blocks", "allocated_pool_blocks",
    "pool_blocks", "hot_slots_used", "hot_slots_capacity", "warm_slots_used", "warm_slots_capacity",
)


def aggregate_memory_metrics(metrics_list) -> dict:
    """tierkv_policy.py:1985-2032: sums plus recomputed ratios."""
    metrics_list = [metrics for metrics in metrics_list if metrics]
    if not metrics_list:
        return TieredKVTensorPool().collect_memory_metrics({})
    out = {key: sum(metrics.get(key, 0) for metrics in metrics_list) for key in _SUMMED_KEYS}
    resident = float(out.get("logical_resident_mb", 0.0))
    dense = float(out.get("logical_dense_equivalent_mb", 0.0))
    out["logical_compression_ratio"] = resident / dense if dense > 0 else 0.0
    out["logical_compression_x"] = dense / resident if resident > 0 else 0.0
    out["pool_utilization"] = out["active_pool_blocks"] / max(float(out["allocated_pool_blocks"]), 1.0)
    out["capacity_utilization"] = out["allocated_pool_blocks"] / max(float(out["pool_blocks"]), 1.0)
    physical_total = float(out.get("physical_total_kv_mb", 0.0))
    out["physical_compression_x"] = dense / physical_total if physical_total > 0 else 0.0
    return out


def reset_global_tierkv() -> None:
    global _GLOBAL_TIERKV_RUNTIME
    if _GLOBAL_TIERKV_RUNTIME is not None:
        _GLOBAL_TIERKV_RUNTIME.reset(release_storage=True)
    _GLOBAL_TIERKV_RUNTIME = None


def get_global_tierkv_runtime():
    return _GLOBAL_TIERKV_RUNTIME

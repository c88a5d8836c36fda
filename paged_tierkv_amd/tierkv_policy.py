"""Tier engine on MI355X -- drop-in for the reference module tierkv_policy.

Public names, constructor arguments, return values, environment variables and
exceptions follow tierkv_policy.py: the codec pair (21-44), the dense
``TieredKVTensorPool`` (53-698, alias ``PhysicalKVPool``),
``CompactTieredKVTensorPool`` (701-1365), ``TierKVPolicyEngine``
(1372-1478), ``LayerRuntimeState`` (1481-1484), the HF ``TieredKVCache``
(1487-1531), ``TieredKVRuntime`` (1534-1912) and the module functions
(1915-2044).  The behaviour the reference's callers and tests observe is kept
exactly -- BlockManager calls, slot ids (LIFO free stacks refilled lowest slot
first), table contents, pool bytes including stale tails, error types and
messages -- and is checked against trajectories the reference itself recorded.

How it is organised here:

* Host half.  Each pool keeps a ledger of ``_Block`` records (tier, slot,
  tokens) and table locations; the reference's per-block dictionaries and
  storage sets are read-only views of it.  Slot storage of every tier is a
  ``_SlotArena`` (LIFO stack for the compact tiers, index coverage for the
  dense pool).  Tier changes are table-driven: ``_TRANSITION_RULES`` gives
  each transition's no-op state and errors, each layout supplies
  ``_present`` / ``_apply``, and ``_RETIER`` maps (assigned, held) state
  pairs to the transition ``sync_storage_states`` needs.  Runtime settings
  come from the ``_SETTINGS`` table of argument/environment precedence.
* Device half.  Every data movement runs in the HIP kernels of
  libtierkv_hip.so (token copies with tail zeroing, the reference codec's
  quantize and dequantize); there is no PyTorch fallback, and a missing
  library raises RuntimeError.  Pool operations queue their copies and launch
  them in batches: a whole prefill is one copy launch plus one quantize
  launch, a whole ``sync_storage_states`` one demote and one promote launch,
  where the reference issues about 20 launches per block.  Queued jobs never
  overlap on a slot (a job that would read or write a slot a queued job
  writes, or write a slot a queued job reads, first launches the queue), so
  batching keeps the sequential semantics.
* Tables keep a host copy; entry writes are queued and pushed with one
  scatter launch when a table is next read (``get_layer_table``,
  ``get_layer_lengths`` or the table attributes).  Host-side reads (lengths,
  metrics) use the host copy, so ``collect_memory_metrics`` does not
  synchronise.
* The policy's ranking runs in the label kernel (one device-to-host copy per
  enforce call instead of one per candidate, tierkv_policy.py:1424, 1462).

Extension (keyword-only): ``warm_format="absmax_i8"`` stores WARM blocks as
int8 codes with fp32 per-(slot, head) scales (``k_zero``/``v_zero`` None);
the default ``"ref_u8"`` is the reference codec.

All tensors are GPU tensors; operations run on the current stream, which must
stay the same across calls on one device.
"""

from __future__ import annotations

import contextlib
import ctypes
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
        self._rows: dict = {}   # (k, layer) -> dev[layer, k] (dev is never replaced)

    def _flat(self, k: int, layer: int, idx: int) -> int:
        return (layer * self.shape[1] + k) * self.shape[2] + idx

    def set(self, k: int, layer: int, idx: int, value: int) -> None:
        layer, idx, value = int(layer), int(idx), int(value)
        if not (0 <= layer < self.shape[0]):
            raise IndexError(f"index {layer} is out of bounds for dimension 0 with size {self.shape[0]}")
        if not (-self.shape[2] <= idx < self.shape[2]):
            raise IndexError(f"index {idx} is out of bounds for dimension 1 with size {self.shape[2]}")
        idx %= self.shape[2]
        if self.host[layer, k, idx] == value:
            return   # the device row already holds it, or a queued entry does
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

    def row_view(self, k: int, layer: int) -> torch.Tensor:
        """One layer's row of table k (queued entries pushed first); the
        decode path asks for the same rows every step, so the views are kept."""
        self.flush()
        v = self._rows.get((k, layer))
        if v is None:
            if not -self.shape[0] <= layer < self.shape[0]:
                raise IndexError(f"index {layer} is out of bounds for dimension 0 with size {self.shape[0]}")
            v = self._rows[(k, layer)] = self.dev[layer, k]
        return v


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
            # A decode step's few jobs ride in the kernel's arguments (the C
            # call copies them, so one host array serves every call).
            jobs = self.__dict__.get("_jobs_host")
            if jobs is None:
                jobs = self._jobs_host = np.zeros((_INLINE_JOBS, 5), np.int32)
            for i, (tok0, count, slot, pos) in enumerate(rows):
                jobs[i] = (0, tok0, count, slot, pos)   # src_seq, src_tok, count, dst_slot, dst_pos
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



# ---------------------------------------------------------------------------
# Host half: what each pool knows about its blocks, where their bytes live,
# and the rules that move a block between tiers.
# ---------------------------------------------------------------------------

@dataclass
class _Block:
    """One stored physical block: its tier, its slot in that tier's storage
    (the compact layout; the dense layout addresses storage by physical id)
    and the tokens it holds."""
    state: int
    slot: int = -1
    length: int = 0


class _SlotArena:
    """Storage rows of one tier, allocated in chunks up to ``limit``.

    Two ways to hand out rows, one per pool layout:

    * ``take`` / ``give`` -- a LIFO stack of free rows (compact tiers).  A
      growth pushes the new rows highest first, so the next ``take`` returns
      the lowest of them; a released row is the next one taken.  Slot ids
      therefore follow tierkv_policy.py:849-915 exactly.
    * ``cover`` -- rows are physical ids; the arena grows to the chunk
      boundary above the requested id (dense pool, tierkv_policy.py:137-185).

    ``on_grow(old, new)`` reallocates the tier's tensors."""

    def __init__(self, limit: int, chunk: int, on_grow, exhausted: str):
        self.limit = int(limit)
        self.chunk = int(chunk)
        self.on_grow = on_grow
        self.exhausted = exhausted
        self.capacity = 0
        self.free: list[int] = []

    def _extend_to(self, new: int) -> None:
        old = self.capacity
        self.on_grow(old, new)
        self.capacity = new
        return old

    def take(self) -> int:
        if not self.free:
            if self.capacity >= self.limit:
                raise RuntimeError(self.exhausted)
            new = min(self.limit, self.capacity + max(1, self.chunk))
            old = self._extend_to(new)
            self.free.extend(range(new - 1, old - 1, -1))
        return int(self.free.pop())

    def give(self, slot: int) -> None:
        if int(slot) >= 0:
            self.free.append(int(slot))

    def cover(self, index: int) -> None:
        if index < self.capacity:
            return
        new = min(self.limit, _ceil_div(index + 1, self.chunk) * self.chunk)
        if new > self.capacity:
            self._extend_to(new)

    def all_free(self) -> None:
        self.free = list(range(self.capacity - 1, -1, -1))

    def drop(self) -> None:
        self.capacity = 0
        self.free = []


# Tier transitions of a stored block (tierkv_policy.py:329-402, 1042-1115):
# the state in which the call does nothing, the error when the block is
# COLD, the error when the source tier does not hold it.
_TRANSITION_RULES = {
    "demote_to_warm": (WARM_STATE, "is not eligible for WARM demotion from COLD storage",
                       "is not present in HOT storage"),
    "promote_to_hot": (HOT_STATE, "is not eligible for HOT promotion from COLD storage",
                       "is not present in WARM storage"),
    "demote_to_cold": (COLD_STATE, None, "is not present in HOT or WARM storage"),
}

# sync_storage_states (tierkv_policy.py:1849-1867): for the state the
# BlockManager now holds and the state the pool holds, the pool call to make
# or the error to raise; pairs not listed need no data movement.
_RETIER = {
    (HOT_STATE, WARM_STATE): "promote_to_hot",
    (HOT_STATE, COLD_STATE): "cannot be promoted from COLD to HOT",
    (WARM_STATE, HOT_STATE): "demote_to_warm",
    (WARM_STATE, COLD_STATE): "cannot be promoted from COLD to WARM",
    (COLD_STATE, HOT_STATE): "demote_to_cold",
    (COLD_STATE, WARM_STATE): "demote_to_cold",
    (COLD_STATE, None): "demote_to_cold",
}


class _PoolBase(_QueuedStorage):
    """What the dense and compact pools share: geometry, the block ledger
    (``_blocks``: stored blocks; ``_where``: table entry of each physical id),
    the tier transitions and the metric arithmetic.  Layout-specific parts:
    ``_present`` / ``_apply`` (transitions), the write paths, the tables."""

    _table_fills: tuple = ()
    _capacity_word = "tensor-pool"

    def __init__(self, num_layers, block_size, max_seq_len, max_blocks_per_layer, pool_blocks, pool_chunk_blocks,
                 warm_format):
        for name, value in (("num_layers", num_layers), ("block_size", block_size), ("max_seq_len", max_seq_len)):
            if value <= 0:
                raise ValueError(f"{name} must be positive.")
        self.num_layers = int(num_layers)
        self.block_size = int(block_size)
        self.max_seq_len = int(max_seq_len)
        self.max_blocks_per_layer = int(max_blocks_per_layer or _ceil_div(max_seq_len, block_size))
        self.pool_blocks = int(pool_blocks or self.num_layers * self.max_blocks_per_layer)
        self.pool_chunk_blocks = int(pool_chunk_blocks)
        self.warm_format = self._check_format(warm_format)
        self.device = None
        self.dtype = torch.float16
        self.kv_heads = None
        self.head_dim = None
        self.full_table_sync_count = 0
        self._tables: _Tables | None = None
        self._blocks: dict[int, _Block] = {}
        self._where: dict[int, tuple[int, int]] = {}
        for name in _POOL_TENSORS:
            setattr(self, name, None)
        self._init_queue()

    # -- the reference's per-block dictionaries and sets, as views ----------
    @property
    def physical_states(self) -> dict:
        return {p: b.state for p, b in self._blocks.items()}

    @property
    def physical_locations(self) -> dict:
        return dict(self._where)

    def _in_tier(self, state: int) -> set:
        return {p for p, b in self._blocks.items() if b.state == state}

    @property
    def hot_storage(self) -> set:
        return self._in_tier(HOT_STATE)

    @property
    def warm_storage(self) -> set:
        return self._in_tier(WARM_STATE)

    @property
    def cold_storage(self) -> set:
        return self._in_tier(COLD_STATE)

    def get_physical_state(self, physical_idx: int) -> int | None:
        b = self._blocks.get(int(physical_idx))
        return None if b is None else b.state

    def _append_token(self, physical_idx: int, pos: int, src_k, src_v) -> None:
        """One token at position pos of a HOT block that has room (the
        runtime's decode-step append)."""
        self._write_hot_range(physical_idx, pos, src_k, src_v, 0, 1)

    def _check_physical_idx(self, physical_idx: int) -> int:
        physical_idx = int(physical_idx)
        if not 0 <= physical_idx < self.pool_blocks:
            raise RuntimeError(f"Physical block {physical_idx} is outside {self._capacity_word} capacity "
                               f"{self.pool_blocks}.")
        return physical_idx

    def _check_entry(self, layer_idx: int, logical_idx: int) -> None:
        if not 0 <= layer_idx < self.num_layers:
            raise ValueError("layer_idx is out of range.")
        if not 0 <= logical_idx < self.max_blocks_per_layer:
            raise RuntimeError(
                f"Logical block {logical_idx} exceeds max_blocks_per_layer={self.max_blocks_per_layer}.")

    def _require_allocated(self) -> None:
        if not self.is_allocated():
            raise RuntimeError(f"{type(self).__name__} has not been allocated yet.")

    def _adopt_geometry(self, key_states: torch.Tensor) -> bool:
        """Take the device / kv_heads / head_dim of the first stored tensor;
        returns whether this call allocated the tables."""
        geometry = (key_states.device, int(key_states.shape[1]), int(key_states.shape[-1]))
        if self._tables is not None:
            if geometry != (self.device, self.kv_heads, self.head_dim):
                raise ValueError("KV tensor geometry changed after tensor-pool allocation.")
            return False
        self.device, self.kv_heads, self.head_dim = geometry
        self._tables = _Tables(self._table_fills, self.num_layers, self.max_blocks_per_layer, self.device)
        return True

    # -- tier transitions ---------------------------------------------------
    def _transition(self, op: str, physical_idx) -> None:
        p = self._check_physical_idx(physical_idx)
        state = self.get_physical_state(p)
        idle, cold_error, missing_error = _TRANSITION_RULES[op]
        if state == idle:
            return
        if cold_error is not None and state == COLD_STATE:
            raise KeyError(f"Physical block {p} {cold_error}.")
        if not self._present(op, p, state):
            raise KeyError(f"Physical block {p} {missing_error}.")
        self._apply(op, p, state)

    def demote_to_warm(self, physical_idx) -> None:
        self._transition("demote_to_warm", physical_idx)

    def promote_to_hot(self, physical_idx) -> None:
        self._transition("promote_to_hot", physical_idx)

    def demote_to_cold(self, physical_idx) -> None:
        self._transition("demote_to_cold", physical_idx)

    def retier(self, physical_idx: int, desired: int) -> None:
        """Bring the pool's copy of a block to the tier the BlockManager
        assigned it (one step of sync_storage_states)."""
        step = _RETIER.get((int(desired), self.get_physical_state(physical_idx)))
        if step is None:
            return
        if step in _TRANSITION_RULES:
            self._transition(step, physical_idx)
        else:
            raise KeyError(f"Physical block {physical_idx} {step}.")

    def store_hot_block(self, physical_idx, k_tensor, v_tensor) -> None:
        self.write_hot_tokens(int(physical_idx), 0, k_tensor, v_tensor)

    def write_hot_tokens(self, physical_idx: int, start: int, key_states: torch.Tensor,
                         value_states: torch.Tensor) -> None:
        p = self._check_physical_idx(physical_idx)
        key_states, value_states = self._coerce_kv(key_states, value_states)
        with self._batch():
            self._write_hot_range(p, start, key_states, value_states, 0, key_states.shape[-2])

    def write_warm_block(self, physical_idx, k_tensor, v_tensor) -> None:
        p = self._check_physical_idx(physical_idx)
        k_tensor, v_tensor = self._coerce_kv(k_tensor, v_tensor)
        with self._batch():
            self._write_warm_range(p, k_tensor, v_tensor, 0, k_tensor.shape[-2])

    def _check_range(self, start: int, tokens: int) -> None:
        if start < 0 or start + tokens > self.block_size:
            raise ValueError("KV write exceeds the physical block capacity.")

    # -- reads --------------------------------------------------------------
    def _hot_rows(self, row: int, length: int):
        self._launch_queue()
        return (self.hot_k_pool[row: row + 1, :, :length, :].contiguous(),
                self.hot_v_pool[row: row + 1, :, :length, :].contiguous())

    def get_dequantized_block(self, physical_idx, state):
        """fp16 K, V of one block as its table state says it is stored
        (tierkv_policy.py:404-448, 1117-1162): a block asked for as HOT but
        held WARM is promoted first; a COLD block reads as zeros."""
        p = self._check_physical_idx(physical_idx)
        if not self.is_allocated():
            raise KeyError(f"Physical block {p} is not present in {self._storage_word} storage.")
        length = self.get_block_length(p)
        held = self.get_physical_state(p)
        if state == COLD_STATE:
            shape = (1, self.kv_heads, length, self.head_dim)
            return (torch.zeros(shape, device=self.device, dtype=torch.float16),
                    torch.zeros(shape, device=self.device, dtype=torch.float16))
        if state not in (HOT_STATE, WARM_STATE):
            raise ValueError(f"Unsupported block state: {state}")
        if held == COLD_STATE:
            raise KeyError(f"Physical block {p} is marked {'HOT' if state == HOT_STATE else 'WARM'} but only "
                           "exists in COLD storage.")
        if state == HOT_STATE:
            if held == WARM_STATE:
                self.promote_to_hot(p)
            return self._hot_rows(self._row_of(p), length)
        if held == HOT_STATE:
            return self._hot_rows(self._row_of(p), length)
        self._launch_queue()
        return self._dequantize_slot(self._row_of(p), length)

    def get_layer_table(self, layer_idx: int):
        self._require_allocated()
        self._before_decode()
        layer_idx = int(layer_idx)
        return self._tables.row_view(self._t_table, layer_idx), self._tables.row_view(self._t_state, layer_idx)

    def get_layer_lengths(self, layer_idx: int):
        self._require_allocated()
        return self._tables.row_view(self._t_len, int(layer_idx))

    def _before_decode(self) -> None:
        pass

    def set_block_state(self, layer_idx: int, logical_idx: int, state: int) -> None:
        self._require_allocated()
        self._tables.set(self._t_state, layer_idx, logical_idx, int(state))

    def _state_settled(self, layer_idx: int, logical_idx: int, physical_idx: int, state: int) -> bool:
        """Whether retier(physical_idx, state) and set_block_state(layer_idx,
        logical_idx, state) would both do nothing now (allocated pools)."""
        return (_RETIER.get((int(state), self.get_physical_state(physical_idx))) is None
                and int(self._tables.host[layer_idx, self._t_state, logical_idx]) == int(state))

    # -- telemetry ----------------------------------------------------------
    def _tensor_bytes_mb(self, names) -> float:
        return sum(self._tensor_mb(getattr(self, n)) for n in names)

    def _physical_mb(self) -> tuple[float, float, float]:
        return (self._tensor_bytes_mb(("hot_k_pool", "hot_v_pool")),
                self._tensor_bytes_mb(("warm_k_pool", "warm_v_pool")),
                self._tensor_bytes_mb(("k_scale", "k_zero", "v_scale", "v_zero")))

    def _tier_counts(self, layer_states: dict):
        """Blocks and tokens per tier over the layers' active blocks, from the
        host copies of the tables; and the active-block figure the layout
        reports."""
        blocks = dict.fromkeys((HOT_STATE, WARM_STATE, COLD_STATE), 0)
        tokens = dict.fromkeys((HOT_STATE, WARM_STATE, COLD_STATE), 0)
        active = 0
        for layer_idx in range(self.num_layers):
            ls = layer_states.get(layer_idx)
            n = int(ls.num_blocks) if ls is not None else 0
            if n <= 0:
                continue
            rows = self._active_rows(layer_idx, n)
            if rows is None:
                continue
            states, lengths = rows
            for s in blocks:
                mask = states == s
                blocks[s] += int(mask.sum())
                tokens[s] += int(lengths[mask].sum())
            active += len(states)
        return blocks, tokens, active

    def collect_memory_metrics(self, layer_states: dict) -> dict:
        """tierkv_policy.py:489-654 / 1193-1317 from the host copies of the
        tables (no device synchronisation)."""
        hot_mb, warm_mb, meta_mb = self._physical_mb()
        out = dict.fromkeys(_TOKEN_KEYS, 0)
        out.update(dict.fromkeys(_MB_KEYS, 0.0))
        out.update(self._capacity_metrics(hot_mb, warm_mb, meta_mb))
        if not self.is_allocated() or self.kv_heads is None or self.head_dim is None:
            return out
        blocks, tokens, active = self._tier_counts(layer_states)
        per_dense = int(self.kv_heads) * int(self.head_dim) * 2 * 2
        per_int8 = int(self.kv_heads) * int(self.head_dim) * 2
        per_meta = int(self.kv_heads) * 4 * 2
        total_tokens = sum(tokens.values())
        mb = float(1024 ** 2)
        hot_b = tokens[HOT_STATE] * per_dense
        warm_b = tokens[WARM_STATE] * per_int8
        meta_b = tokens[WARM_STATE] * per_meta
        dense_b = total_tokens * per_dense
        resident_b = hot_b + warm_b + meta_b
        out.update({
            "hot_blocks": blocks[HOT_STATE], "warm_blocks": blocks[WARM_STATE], "cold_blocks": blocks[COLD_STATE],
            "hot_tokens": tokens[HOT_STATE], "warm_tokens": tokens[WARM_STATE], "cold_tokens": tokens[COLD_STATE],
            "active_tokens": total_tokens,
            "logical_hot_mb": hot_b / mb, "logical_warm_mb": warm_b / mb, "logical_warm_meta_mb": meta_b / mb,
            "logical_cold_evicted_mb": tokens[COLD_STATE] * per_dense / mb,
            "logical_dense_equivalent_mb": dense_b / mb, "logical_resident_mb": resident_b / mb,
        })
        out.update(self._usage_metrics(blocks, active, dense_b, resident_b, hot_mb + warm_mb + meta_mb))
        return out

    # -- lifecycle ------------------------------------------------------------
    def _forget_blocks(self) -> None:
        self._blocks.clear()
        self._where.clear()
        self.full_table_sync_count = 0

    def clear(self) -> None:
        """Forget every block; tensors and capacity stay (tierkv_policy.py:662-674, 1319-1334)."""
        self._launch_queue()
        if self.is_allocated():
            self._tables.reset()
        self._forget_blocks()
        self._reset_rows()

    def release(self) -> None:
        """Drop every tensor and forget every block."""
        self._launch_queue()
        for name in _POOL_TENSORS:
            setattr(self, name, None)
        self._tables = None
        self.device = self.kv_heads = self.head_dim = None
        self._forget_blocks()
        self._drop_rows()


_POOL_TENSORS = ("hot_k_pool", "hot_v_pool", "warm_k_pool", "warm_v_pool", "k_scale", "k_zero", "v_scale", "v_zero")
_TOKEN_KEYS = ("hot_blocks", "warm_blocks", "cold_blocks", "hot_tokens", "warm_tokens", "cold_tokens",
               "active_tokens")
_MB_KEYS = ("logical_hot_mb", "logical_warm_mb", "logical_warm_meta_mb", "logical_cold_evicted_mb",
            "logical_dense_equivalent_mb", "logical_resident_mb", "logical_compression_ratio",
            "logical_compression_x")


# ---------------------------------------------------------------------------
# Dense layout (tierkv_policy.py:53-698): a block's physical id is its row
# in every tier's tensors; the table holds the physical id.
# ---------------------------------------------------------------------------

class TieredKVTensorPool(_PoolBase):
    _demote_pads_tail = True       # demote_to_warm zero-pads the tail (350-356)
    _stage_pads_tail = False       # write_warm_block copies [:length] only (292-312)
    _table_fills = (-1, COLD_STATE, 0)
    _t_table, _t_state, _t_len = 0, 1, 2
    _storage_word = "tensor-pool"

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
        super().__init__(num_layers, block_size, max_seq_len, max_blocks_per_layer, pool_blocks, pool_chunk_blocks,
                         warm_format)
        if self.pool_chunk_blocks <= 0:
            raise ValueError("pool_chunk_blocks must be positive.")
        self._rows = _SlotArena(self.pool_blocks, self.pool_chunk_blocks, self._grow_rows, "")
        self._lengths: _Vector | None = None        # tokens per physical id

    # Table views (queued entries are pushed first).
    @property
    def block_tables(self):
        return None if self._tables is None else self._tables.view(self._t_table)

    @property
    def block_states(self):
        return None if self._tables is None else self._tables.view(self._t_state)

    @property
    def logical_block_lengths(self):
        return None if self._tables is None else self._tables.view(self._t_len)

    @property
    def block_lengths(self):
        return None if self._lengths is None else self._lengths.tensor()

    @property
    def allocated_pool_blocks(self) -> int:
        return self._rows.capacity

    def is_allocated(self) -> bool:
        return self.hot_k_pool is not None

    def _row_of(self, physical_idx: int) -> int:
        return physical_idx

    def _grow_rows(self, old: int, new: int) -> None:
        self._launch_queue()
        shape = (new, self.kv_heads, self.block_size, self.head_dim)
        for name, dtype in (("hot_k_pool", torch.float16), ("hot_v_pool", torch.float16),
                            ("warm_k_pool", self._warm_dtype()), ("warm_v_pool", self._warm_dtype())):
            setattr(self, name, self._grow_copy(getattr(self, name), torch.zeros(shape, device=self.device,
                                                                                 dtype=dtype), old))
        for name, fresh in (("k_scale", self._new_scale(new, 1)), ("k_zero", self._new_zero_point(new)),
                            ("v_scale", self._new_scale(new, 1)), ("v_zero", self._new_zero_point(new))):
            setattr(self, name, self._grow_copy(getattr(self, name), fresh, old))
        if self._lengths is None:
            self._lengths = _Vector(new, self.device)
        else:
            self._lengths.grow(new)

    def _reserve(self, key_states: torch.Tensor, physical_idx: int) -> None:
        """Tables on the first store, rows up to the chunk above physical_idx."""
        if key_states.ndim != 4:
            raise ValueError("KV tensors must have shape [1, kv_heads, tokens, head_dim].")
        if key_states.shape[0] != 1:
            raise ValueError("TieredKVTensorPool currently supports batch size 1 only.")
        self._adopt_geometry(key_states)
        self._rows.cover(physical_idx)

    def get_block_length(self, physical_idx: int) -> int:
        p = self._check_physical_idx(physical_idx)
        if self._lengths is None or p >= self._rows.capacity:
            return 0
        return int(self._lengths.host[p])

    def _record(self, physical_idx: int, state: int, length: int | None = None) -> None:
        """A block's new tier (and token count), mirrored into its table row."""
        if length is not None:
            self._lengths.set(physical_idx, length)
            where = self._where.get(physical_idx)
            if where is not None and self._tables is not None:
                self._tables.set(self._t_len, where[0], where[1], length)
        self._blocks[physical_idx] = _Block(state)

    def _write_hot_range(self, physical_idx, start, src_k, src_v, tok0, tokens) -> None:
        self._reserve(src_k, physical_idx)
        start, tokens = int(start), int(tokens)
        self._check_range(start, tokens)
        self._queue_write(src_k, src_v, tok0, tokens, physical_idx, start)
        self._record(physical_idx, HOT_STATE, start + tokens)

    def _write_warm_range(self, physical_idx, src_k, src_v, tok0, length) -> None:
        self._reserve(src_k, physical_idx)
        self._queue_stage(src_k, src_v, tok0, length, physical_idx)
        self._record(physical_idx, WARM_STATE, int(length))

    def register_cold_block(self, physical_idx, length: int) -> None:
        p = self._check_physical_idx(physical_idx)
        self._record(p, COLD_STATE, int(length) if self._lengths is not None else None)

    def _present(self, op: str, p: int, state) -> bool:
        if op == "promote_to_hot":
            return state == WARM_STATE
        return self.is_allocated() and self.get_block_length(p) > 0

    def _apply(self, op: str, p: int, state) -> None:
        if op == "demote_to_warm":
            self._queue_demote(p, p, self.get_block_length(p))
            self._record(p, WARM_STATE)
        elif op == "promote_to_hot":
            self._queue_promote(p, p, self.get_block_length(p))
            self._record(p, HOT_STATE)
        else:
            self._record(p, COLD_STATE)

    def _write_entry(self, layer_idx: int, logical_idx: int, physical_idx: int, state: int) -> None:
        self._tables.set(self._t_table, layer_idx, logical_idx, physical_idx)
        self._tables.set(self._t_state, layer_idx, logical_idx, int(state))
        self._tables.set(self._t_len, layer_idx, logical_idx, int(self._lengths.host[physical_idx]))
        self._where[physical_idx] = (layer_idx, logical_idx)

    def _check_row(self, physical_idx: int) -> None:
        # the reference indexes its per-physical-id lengths tensor here
        n = self._lengths.host.size
        if not 0 <= physical_idx < n:
            raise IndexError(f"index {physical_idx} is out of bounds for dimension 0 with size {n}")

    def set_block_entry(self, layer_idx: int, logical_idx: int, physical_idx: int, state: int) -> None:
        self._require_allocated()
        layer_idx, logical_idx = int(layer_idx), int(logical_idx)
        physical_idx = self._check_physical_idx(physical_idx)
        self._check_entry(layer_idx, logical_idx)
        self._check_row(physical_idx)
        self._write_entry(layer_idx, logical_idx, physical_idx, state)

    def sync_gpu_block_tables(self, layer_idx: int, physical_indices, states) -> None:
        """Rewrite one layer's table rows from the BlockManager's lists (tierkv_policy.py:450-477)."""
        if not self.is_allocated():
            return
        self.full_table_sync_count += 1
        layer_idx = int(layer_idx)
        if not 0 <= layer_idx < self.num_layers:
            raise ValueError("layer_idx is out of range.")
        if len(physical_indices) > self.max_blocks_per_layer:
            raise RuntimeError(f"Layer {layer_idx} has {len(physical_indices)} blocks, exceeding "
                               f"max_blocks_per_layer={self.max_blocks_per_layer}.")
        if len(physical_indices) != len(states):
            raise ValueError("Block table and state table lengths must match.")
        if any(not 0 <= int(p) < self._lengths.host.size for p in physical_indices):
            raise IndexError("index out of range in self")
        for k, fill in enumerate(self._table_fills):
            self._tables.fill_row(k, layer_idx, fill)
        for logical_idx, (p, s) in enumerate(zip(physical_indices, states)):
            self._write_entry(layer_idx, logical_idx, int(p), s)

    def _active_rows(self, layer_idx: int, n: int):
        table = self._tables.row(self._t_table, layer_idx)[:n]
        keep = table >= 0
        if not keep.any():
            return None
        lengths = np.maximum(self._lengths.host[table[keep]], 0).astype(np.int64)
        return self._tables.row(self._t_state, layer_idx)[:n][keep], lengths

    def _capacity_metrics(self, hot_mb, warm_mb, meta_mb) -> dict:
        cap = int(self._rows.capacity)
        return {
            "physical_hot_pool_mb": 0.0, "physical_warm_pool_mb": 0.0, "physical_warm_meta_mb": 0.0,
            "physical_total_kv_mb": 0.0, "physical_compression_x": 0.0,
            "hot_slots_used": 0, "hot_slots_capacity": cap, "warm_slots_used": 0, "warm_slots_capacity": cap,
            "active_pool_blocks": 0, "allocated_pool_blocks": cap, "pool_blocks": int(self.pool_blocks),
            "pool_utilization": 0.0, "capacity_utilization": float(cap) / max(float(self.pool_blocks), 1.0),
        }

    def _usage_metrics(self, blocks, active, dense_b, resident_b, total_mb) -> dict:
        hot_mb, warm_mb, meta_mb = self._physical_mb()
        dense_mb = dense_b / float(1024 ** 2)
        return {
            "logical_compression_ratio": resident_b / dense_b if dense_b > 0 else 0.0,
            "logical_compression_x": dense_b / resident_b if resident_b > 0 else 0.0,
            "active_pool_blocks": active,
            "pool_utilization": active / max(float(self._rows.capacity), 1.0),
            "physical_hot_pool_mb": hot_mb, "physical_warm_pool_mb": warm_mb, "physical_warm_meta_mb": meta_mb,
            "physical_total_kv_mb": total_mb,
            "physical_compression_x": dense_mb / max(total_mb, 1e-12) if dense_mb > 0 else 0.0,
            "hot_slots_used": blocks[HOT_STATE], "warm_slots_used": blocks[WARM_STATE],
        }

    def _reset_rows(self) -> None:
        if self._lengths is not None and self.is_allocated():
            self._lengths.zero()

    def _drop_rows(self) -> None:
        self._lengths = None
        self._rows.drop()


# ---------------------------------------------------------------------------
# Compact layout (tierkv_policy.py:701-1365): HOT and WARM keep their own slot
# storage; the table holds the tier-specific slot (-1 for COLD) beside the
# physical id.
# ---------------------------------------------------------------------------

class CompactTieredKVTensorPool(_PoolBase):
    _table_fills = (-1, -1, COLD_STATE, 0)
    _t_phys, _t_table, _t_state, _t_len = 0, 1, 2, 3
    _capacity_word = "tensor-pool metadata"
    _storage_word = "compact tensor-pool"

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
        super().__init__(num_layers, block_size, max_seq_len, max_blocks_per_layer, pool_blocks, pool_chunk_blocks,
                         warm_format)
        self.max_hot_slots = int(self.pool_blocks if max_hot_slots is None else max_hot_slots)
        self.max_warm_slots = int(self.pool_blocks if max_warm_slots is None else max_warm_slots)
        self.hot_chunk_slots = int(hot_chunk_slots or self.pool_chunk_blocks)
        self.warm_chunk_slots = int(warm_chunk_slots or self.pool_chunk_blocks)
        if min(self.max_hot_slots, self.max_warm_slots) < 0:
            raise ValueError("max_hot_slots and max_warm_slots must be non-negative.")
        self._hot = _SlotArena(self.max_hot_slots, self.hot_chunk_slots, self._grow_hot,
                               "No HOT slots available in compact TierKV pool.")
        self._warm = _SlotArena(self.max_warm_slots, self.warm_chunk_slots, self._grow_warm,
                                "No WARM slots available in compact TierKV pool.")

    # Views of the slot arenas and the ledger in the reference's names.
    @property
    def hot_free_slots(self) -> list:
        return self._hot.free

    @property
    def warm_free_slots(self) -> list:
        return self._warm.free

    @property
    def allocated_hot_slots(self) -> int:
        return self._hot.capacity

    @property
    def allocated_warm_slots(self) -> int:
        return self._warm.capacity

    @property
    def allocated_pool_blocks(self) -> int:
        return max(self._hot.capacity, self._warm.capacity)

    @property
    def physical_slots(self) -> dict:
        return {p: b.slot for p, b in self._blocks.items()}

    @property
    def physical_lengths(self) -> dict:
        return {p: b.length for p, b in self._blocks.items()}

    # Table views (queued entries are pushed first).
    @property
    def physical_block_tables(self):
        return None if self._tables is None else self._tables.view(self._t_phys)

    @property
    def block_slot_indices(self):
        return None if self._tables is None else self._tables.view(self._t_table)

    block_tables = block_slot_indices

    @property
    def block_states(self):
        return None if self._tables is None else self._tables.view(self._t_state)

    @property
    def block_lengths(self):
        return None if self._tables is None else self._tables.view(self._t_len)

    def is_allocated(self) -> bool:
        return self._tables is not None

    def get_block_length(self, physical_idx: int) -> int:
        b = self._blocks.get(int(physical_idx))
        return 0 if b is None else b.length

    def _row_of(self, physical_idx: int) -> int:
        return self._blocks[physical_idx].slot

    def _kv_rows(self, n: int, dtype):
        return torch.zeros((n, self.kv_heads, self.block_size, self.head_dim), device=self.device, dtype=dtype)

    def _grow_hot(self, old: int, new: int) -> None:
        self._launch_queue()
        self.hot_k_pool = self._grow_copy(self.hot_k_pool, self._kv_rows(new, torch.float16), old)
        self.hot_v_pool = self._grow_copy(self.hot_v_pool, self._kv_rows(new, torch.float16), old)

    def _grow_warm(self, old: int, new: int) -> None:
        self._launch_queue()
        self.warm_k_pool = self._grow_copy(self.warm_k_pool, self._kv_rows(new, self._warm_dtype()), old)
        self.warm_v_pool = self._grow_copy(self.warm_v_pool, self._kv_rows(new, self._warm_dtype()), old)
        self.k_scale = self._grow_copy(self.k_scale, self._new_scale(new, 1), old)
        self.k_zero = self._grow_copy(self.k_zero, self._new_zero_point(new), old)
        self.v_scale = self._grow_copy(self.v_scale, self._new_scale(new, 1), old)
        self.v_zero = self._grow_copy(self.v_zero, self._new_zero_point(new), old)

    def _before_decode(self) -> None:
        """One-row tensors for a tier that has never stored a block, so the
        decode kernel always receives valid pointers (tierkv_policy.py:814-826);
        the tier's first growth replaces them."""
        if self.hot_k_pool is None:
            self.hot_k_pool, self.hot_v_pool = self._kv_rows(1, torch.float16), self._kv_rows(1, torch.float16)
        if self.warm_k_pool is None:
            self.warm_k_pool, self.warm_v_pool = (self._kv_rows(1, self._warm_dtype()),
                                                  self._kv_rows(1, self._warm_dtype()))
            self.k_scale, self.v_scale = self._new_scale(1, 1), self._new_scale(1, 1)
            self.k_zero, self.v_zero = self._new_zero_point(1), self._new_zero_point(1)

    def _arena(self, state: int) -> _SlotArena | None:
        return self._hot if state == HOT_STATE else self._warm if state == WARM_STATE else None

    def _release_slot(self, physical_idx: int) -> None:
        """Give the block's current slot back to its tier's stack."""
        b = self._blocks.get(physical_idx)
        if b is not None and self._arena(b.state) is not None:
            self._arena(b.state).give(b.slot)

    def _record(self, physical_idx: int, state: int, slot: int, length: int) -> None:
        """A block's new tier, slot and token count, mirrored into its table row
        (tierkv_policy.py:917-926)."""
        self._blocks[physical_idx] = _Block(int(state), int(slot), int(length))
        where = self._where.get(physical_idx)
        if where is not None and self._tables is not None:
            for column, value in ((self._t_state, state), (self._t_table, slot), (self._t_len, length)):
                self._tables.set(column, where[0], where[1], int(value))

    def _write_hot_range(self, physical_idx, start, src_k, src_v, tok0, tokens) -> None:
        if src_k.ndim != 4 or src_k.shape[0] != 1:
            raise ValueError("KV tensors must have shape [1, kv_heads, tokens, head_dim].")
        self._adopt_geometry(src_k)
        start, tokens = int(start), int(tokens)
        self._check_range(start, tokens)
        held = self.get_physical_state(physical_idx)
        if held == COLD_STATE:
            raise KeyError(f"Physical block {physical_idx} is COLD and cannot be promoted.")
        if held == WARM_STATE:
            self.promote_to_hot(physical_idx)
        slot = self._hot.take() if held is None else self._blocks[physical_idx].slot
        self._queue_write(src_k, src_v, tok0, tokens, slot, start)
        self._record(physical_idx, HOT_STATE, slot, start + tokens)

    def _append_token(self, physical_idx: int, pos: int, src_k, src_v) -> None:
        """_write_hot_range's effect for one token into a HOT block with room
        and nothing queued: the write launch, the block's new length and its
        table entry; anything else takes the general path."""
        b = self._blocks.get(physical_idx)
        if (b is None or b.state != HOT_STATE or self._depth or self._q_write or self._q_stage or self._q_dem
                or self._q_pro or not 0 <= pos < self.block_size or self._tables is None
                or src_k.shape[1] != self.kv_heads or src_k.shape[-1] != self.head_dim
                or src_k.device != self.device):
            self._write_hot_range(physical_idx, pos, src_k, src_v, 0, 1)
            return
        self._launch_writes(_lib.lib(), src_k, src_v, [(0, 1, b.slot, pos)], self.hot_k_pool, self.hot_v_pool,
                            _lib.stream_of(self.device))
        self._blocks[physical_idx] = _Block(HOT_STATE, b.slot, pos + 1)
        where = self._where.get(physical_idx)
        if where is not None:
            self._tables.set(self._t_len, where[0], where[1], pos + 1)

    def _fused_inputs_ok(self, query_states, key_states, value_states, new_pairs: int) -> bool:
        """_decode_step's conditions that do not depend on the block: nothing
        queued, room in the inline table writes for new_pairs more entries,
        one contiguous fp16 token per kv head in the pool's geometry."""
        tables = self._tables
        if (tables is None or self._depth or self._q_write or self._q_stage or self._q_dem or self._q_pro
                or len(tables.pending) + new_pairs > _INLINE_PAIRS - 1):
            return False
        return not (key_states.dtype != torch.float16 or value_states.dtype != torch.float16 or key_states.ndim != 4
                    or key_states.shape != value_states.shape or key_states.shape[0] != 1
                    or key_states.shape[1] != self.kv_heads or key_states.shape[-1] != self.head_dim
                    or key_states.shape[2] != 1 or not key_states.is_cuda or key_states.device != self.device
                    or not key_states.is_contiguous() or not value_states.is_contiguous()
                    or not query_states.is_contiguous())

    def _open_hot(self, physical_idx: int, src_k) -> None:
        """_write_hot_range's placement of a new block's first token for a
        decode step that writes the token in its own launch: the HOT slot and
        the ledger entry (one token), mirrored into the tables as the general
        path does, with no queued write."""
        self._adopt_geometry(src_k)
        held = self.get_physical_state(physical_idx)
        if held == COLD_STATE:
            raise KeyError(f"Physical block {physical_idx} is COLD and cannot be promoted.")
        if held == WARM_STATE:
            self.promote_to_hot(physical_idx)
        slot = self._hot.take() if held is None else self._blocks[physical_idx].slot
        self._record(physical_idx, HOT_STATE, slot, 1)

    def _decode_step(self, layer_idx: int, physical_idx: int, pos: int, num_blocks: int, query_states, key_states,
                     value_states, num_key_value_groups: int, scaling: float, cache: dict):
        """_append_token's token write and table update, the queued table
        entries and the layer's decode launch as one tierkv_decode_step call.
        Returns the attention output, or None (nothing done) when the step is
        not the plain case: an fp16 token into a HOT block with room, nothing
        queued, at most 16 table entries to push, tensors as the cached launch
        was validated for."""
        from . import tierkv_hip
        b = self._blocks.get(physical_idx)
        where = self._where.get(physical_idx)
        tables = self._tables
        if (b is None or b.state != HOT_STATE or where is None or not 0 <= pos < self.block_size
                or not self._fused_inputs_ok(query_states, key_states, value_states, 0)):
            return None
        self._before_decode()
        # The cached launch holds the tensors it was bound to, so a replaced
        # pool (growth) is a different object and binds anew.
        tensors = (self.hot_k_pool, self.hot_v_pool, self.warm_k_pool, self.warm_v_pool, self.k_scale, self.k_zero,
                   self.v_scale, self.v_zero)
        key = (query_states.dtype, tuple(query_states.shape), int(num_key_value_groups), float(scaling))
        entry = cache.get(layer_idx)
        if entry is None or entry[0] != key or any(a is not t for a, t in zip(entry[1], tensors)):
            # Validate the launch once with the ordinary binding (it raises
            # what tierkv_decode_attention raises) and keep its arguments.
            args = tierkv_hip._bind(
                query_states, tables.row_view(self._t_table, layer_idx), tables.row_view(self._t_state, layer_idx),
                tables.row_view(self._t_len, layer_idx), self.hot_k_pool, self.hot_v_pool, self.warm_k_pool,
                self.warm_v_pool, self.k_scale, self.k_zero, self.v_scale, self.v_zero, num_blocks,
                num_key_value_groups, scaling, False, cold_mode="zero_logit")[0]
            st = _lib.DecodeStep()
            (_, st.query_dtype, _, _, st.block_table, st.block_states, st.block_lengths, st.table_stride, _, _,
             st.hot_k, st.hot_v, st.hot_slots, st.warm_k, st.warm_v, st.warm_slots, st.k_scale, st.k_zero,
             st.v_scale, st.v_zero, st.warm_format, st.cold_mode, st.batch, st.num_heads, st.num_kv_heads,
             st.block_size, st.head_dim, st.scaling, st.splits_hint) = args[:29]
            st.table_dst = _lib.ptr(tables.dev)
            st.table_len = tables.dev.numel()
            st.src_seqs, st.n_jobs, st.zero_tail = 1, 1, 0
            st.jobs[0][0], st.jobs[0][1], st.jobs[0][2] = 0, 0, 1   # src_seq, src_tok, count
            entry = cache[layer_idx] = (key, tensors, st, {}, ctypes.byref(st), st.jobs[0])
        st, needs, st_ref, job = entry[2], entry[3], entry[4], entry[5]
        n = int(num_blocks)
        if not 0 < n <= st.table_stride:
            return None
        need = needs.get(n)
        lib = _lib.lib()
        if need is None:
            need = needs[n] = lib.tierkv_decode_workspace_bytes(st.batch, st.num_heads, st.num_kv_heads, n,
                                                                st.block_size, st.head_dim, 0, st.splits_hint)
            if need < 0:
                return None
        ws = tierkv_hip.stream_workspace(self.device)
        ws.reserve(need)
        out = torch.empty((1, 1, st.num_heads, st.head_dim), device=self.device, dtype=query_states.dtype)
        # Host state first, as the general path records it before launching.
        self._blocks[physical_idx] = _Block(HOT_STATE, b.slot, pos + 1)
        tables.set(self._t_len, where[0], where[1], pos + 1)
        pending = tables.pending
        sent = dict(pending)
        for i, (flat, value) in enumerate(sent.items()):
            st.pairs[i][0], st.pairs[i][1] = flat, value
        st.n_pairs = len(sent)
        pending.clear()
        st.src_k, st.src_v = key_states.data_ptr(), value_states.data_ptr()
        st.src_tokens = key_states.shape[2]
        job[3], job[4] = b.slot, pos
        st.query, st.out, st.num_blocks = query_states.data_ptr(), out.data_ptr(), n
        st.workspace, st.workspace_bytes = ws.data_ptr(), ws.nbytes
        rc = lib.tierkv_decode_step(st_ref, _lib.stream_of(self.device))
        if rc != _lib.TIERKV_OK:
            # A refused step queued nothing on the device (its checks run
            # before its first launch): the ledger entry and the block's
            # length return to what they were, and the table entries go back
            # to the queue, so host and device tables agree once it is
            # flushed.
            self._blocks[physical_idx] = b
            pending.update(sent)
            tables.set(self._t_len, where[0], where[1], b.length)
            _lib.check(rc, "tierkv_decode_step")
        return out

    def _write_warm_range(self, physical_idx, src_k, src_v, tok0, length) -> None:
        if src_k.ndim != 4 or src_k.shape[0] != 1:
            raise ValueError("KV tensors must have shape [1, kv_heads, tokens, head_dim].")
        self._adopt_geometry(src_k)
        if self.get_physical_state(physical_idx) == COLD_STATE:
            raise KeyError(f"Physical block {physical_idx} is COLD and cannot be promoted.")
        self._release_slot(physical_idx)
        slot = self._warm.take()
        self._queue_stage(src_k, src_v, tok0, length, slot)
        self._record(physical_idx, WARM_STATE, slot, int(length))

    def register_cold_block(self, physical_idx, length: int) -> None:
        p = self._check_physical_idx(physical_idx)
        self._release_slot(p)
        self._record(p, COLD_STATE, -1, int(length))

    def _present(self, op: str, p: int, state) -> bool:
        return state in {"demote_to_warm": (HOT_STATE,), "promote_to_hot": (WARM_STATE,),
                         "demote_to_cold": (HOT_STATE, WARM_STATE)}[op]

    def _apply(self, op: str, p: int, state) -> None:
        b = self._blocks[p]
        if op == "demote_to_cold":
            self._release_slot(p)
            self._record(p, COLD_STATE, -1, b.length)
            return
        # The destination slot is taken before the source slot is released.
        if op == "demote_to_warm":
            dst = self._warm.take()
            self._queue_demote(b.slot, dst, b.length)
            self._hot.give(b.slot)
            self._record(p, WARM_STATE, dst, b.length)
        else:
            dst = self._hot.take()
            self._queue_promote(b.slot, dst, b.length)
            self._warm.give(b.slot)
            self._record(p, HOT_STATE, dst, b.length)

    def set_block_entry(self, layer_idx: int, logical_idx: int, physical_idx: int, state: int) -> None:
        self._require_allocated()
        layer_idx, logical_idx = int(layer_idx), int(logical_idx)
        physical_idx = self._check_physical_idx(physical_idx)
        self._check_entry(layer_idx, logical_idx)
        self._where[physical_idx] = (layer_idx, logical_idx)
        b = self._blocks.get(physical_idx)
        for column, value in ((self._t_phys, physical_idx), (self._t_state, state),
                              (self._t_table, -1 if b is None else b.slot), (self._t_len, 0 if b is None else b.length)):
            self._tables.set(column, layer_idx, logical_idx, int(value))

    def sync_gpu_block_tables(self, layer_idx: int, physical_indices, states) -> None:
        """Rewrite one layer's table rows from the BlockManager's lists (tierkv_policy.py:1164-1174)."""
        if not self.is_allocated():
            return
        self.full_table_sync_count += 1
        layer_idx = int(layer_idx)
        for k, fill in enumerate(self._table_fills):
            self._tables.fill_row(k, layer_idx, fill)
        for logical_idx, (p, s) in enumerate(zip(physical_indices, states)):
            self.set_block_entry(layer_idx, logical_idx, int(p), int(s))

    def _active_rows(self, layer_idx: int, n: int):
        return (self._tables.row(self._t_state, layer_idx)[:n],
                self._tables.row(self._t_len, layer_idx)[:n].astype(np.int64))

    def _capacity_metrics(self, hot_mb, warm_mb, meta_mb) -> dict:
        return {
            "active_pool_blocks": 0, "allocated_pool_blocks": int(self.allocated_pool_blocks),
            "pool_blocks": int(self.pool_blocks), "pool_utilization": 0.0, "capacity_utilization": 0.0,
            "physical_hot_pool_mb": hot_mb, "physical_warm_pool_mb": warm_mb, "physical_warm_meta_mb": meta_mb,
            "physical_total_kv_mb": hot_mb + warm_mb + meta_mb, "physical_compression_x": 0.0,
            "hot_slots_used": len(self.hot_storage), "hot_slots_capacity": int(self._hot.capacity),
            "warm_slots_used": len(self.warm_storage), "warm_slots_capacity": int(self._warm.capacity),
        }

    def _usage_metrics(self, blocks, active, dense_b, resident_b, total_mb) -> dict:
        mb = float(1024 ** 2)
        dense_mb, resident_mb = dense_b / mb, resident_b / mb
        resident_blocks = blocks[HOT_STATE] + blocks[WARM_STATE]
        allocated = self._hot.capacity + self._warm.capacity
        limit = self.max_hot_slots + self.max_warm_slots
        return {
            "logical_compression_ratio": resident_mb / dense_mb if dense_mb > 0 else 0.0,
            "logical_compression_x": dense_mb / resident_mb if resident_mb > 0 else 0.0,
            "active_pool_blocks": resident_blocks, "allocated_pool_blocks": int(allocated), "pool_blocks": int(limit),
            "pool_utilization": resident_blocks / max(float(allocated), 1.0),
            "capacity_utilization": allocated / max(float(limit), 1.0),
            "physical_compression_x": dense_mb / total_mb if total_mb > 0 else 0.0,
        }

    def _reset_rows(self) -> None:
        self._hot.all_free()
        self._warm.all_free()

    def _drop_rows(self) -> None:
        self._hot.drop()
        self._warm.drop()


# The reference keeps the old public name for its tests (tierkv_policy.py:1368-1369).
PhysicalKVPool = TieredKVTensorPool

# ---------------------------------------------------------------------------
# Policy engine (tierkv_policy.py:1372-1478): scores in, BlockManager states
# out; the ranking runs in the label kernel.
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

    def _relabel(self, seq_id, block_scores, hot_budget, warm_budget, mode, demoted_state=WARM_STATE) -> None:
        """Rank the sequence's blocks and write the states that change into
        the BlockManager (tierkv_policy.py:1391-1477).  Sequences of at most
        two blocks are all HOT (the first and last blocks are reserved)."""
        current = self.block_manager.get_states(seq_id)
        n = len(self.block_manager.get_physical_indices(seq_id))
        if n == 0:
            return
        checks = ((mode == "hot_warm" and demoted_state not in (WARM_STATE, COLD_STATE),
                   "demoted_state must be WARM_STATE or COLD_STATE."),
                  (block_scores.ndim != 1, "block_scores must be a 1D tensor."),
                  (block_scores.ndim == 1 and len(block_scores) != n,
                   "block_scores length must match the allocated block count."),
                  (len(current) != n, "Block state table is inconsistent with physical index table."))
        for failed, message in checks:
            if failed:
                raise ValueError(message)
        wanted = ([HOT_STATE] * n if n <= 2
                  else _labels(block_scores, current, hot_budget, warm_budget, mode, demoted_state))
        for logical_idx, (have, want) in enumerate(zip(current, wanted)):
            if have != want:
                self.block_manager.update_block_state(seq_id, logical_idx, int(want))

    def enforce_budget(self, seq_id: int, block_scores: torch.Tensor, hot_budget: int,
                       demoted_state: int = WARM_STATE):
        self._relabel(seq_id, block_scores, hot_budget, 0, "hot_warm", demoted_state)

    def enforce_tiered_budget(self, seq_id: int, block_scores: torch.Tensor, hot_budget: int, warm_budget: int):
        self._relabel(seq_id, block_scores, hot_budget, warm_budget, "hot_warm_cold")


@dataclass
class LayerRuntimeState:
    """A layer's block count and the block still taking appended tokens."""
    open_physical_idx: int | None = None
    open_token_count: int = 0
    num_blocks: int = 0


class TieredKVCache(HFCache):
    """The HF cache object of a tiered runtime (tierkv_policy.py:1487-1531):
    it counts the committed tokens; the KV itself lives in the runtime.  The
    beam and crop hooks are no-ops."""

    is_compileable = False

    def __init__(self, runtime):
        self.runtime = runtime
        self.is_tierkv_cache = True
        self.reset()

    def begin_forward(self, query_length: int) -> None:
        self.pending_query_length = int(query_length)
        self.runtime.begin_forward(query_length)

    def finish_forward(self) -> None:
        self.committed_seq_len, self.pending_query_length = self.committed_seq_len + self.pending_query_length, 0
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

def _flag(value) -> bool:
    return str(value).lower() in ("1", "true", "yes", "on")


# Runtime settings and where they come from (tierkv_policy.py:1551-1575):
# (name, environment variable, the environment overrides the argument?,
#  parse, accepted values or a predicate, error message).  Settings the
# environment does not override read it only when the argument is missing.
_SETTINGS = (
    ("attention_backend", "TIERKV_ATTENTION_BACKEND", False, str, ("eager", "triton"),
     'attention_backend must be "eager" or "triton".'),
    ("policy_interval", "TIERKV_POLICY_INTERVAL", False, int, lambda v: v > 0, "policy_interval must be positive."),
    ("pool_chunk_blocks", "TIERKV_POOL_CHUNK_BLOCKS", True, int, lambda v: v > 0,
     "pool_chunk_blocks must be positive."),
    ("policy_on_new_block", "TIERKV_POLICY_ON_NEW_BLOCK", True, _flag, None, None),
    ("score_accumulation_mode", "TIERKV_SCORE_ACCUMULATION_MODE", True, str, ("policy_ticks", "every_step"),
     'score_accumulation_mode must be "policy_ticks" or "every_step".'),
    ("policy_mode", "TIERKV_POLICY_MODE", True, str, ("hot_only", "hot_warm", "hot_warm_cold"),
     'policy_mode must be "hot_only", "hot_warm", or "hot_warm_cold".'),
    ("warm_budget", "TIERKV_WARM_BUDGET", True, int, lambda v: v >= 0, "warm_budget must be non-negative."),
    ("pool_layout", "TIERKV_POOL_LAYOUT", True, str, ("compact", "dense"), 'pool_layout must be "compact" or "dense".'),
)
# Fallbacks when neither the argument nor the environment gives a value.
_FALLBACK = {"attention_backend": "triton", "policy_interval": 16, "pool_layout": "compact"}


def _resolve_settings(given: dict) -> dict:
    out = {}
    for name, var, env_first, parse, accepted, message in _SETTINGS:
        arg = given[name]
        missing = arg is None or (name in ("attention_backend", "pool_layout") and not arg)
        if env_first and var in os.environ:
            raw = os.environ[var]
        elif not missing:
            raw = arg
        else:
            raw = os.environ.get(var, _FALLBACK.get(name))
        value = parse(raw)
        ok = True if accepted is None else (accepted(value) if callable(accepted) else value in accepted)
        if not ok:
            raise ValueError(message)
        out[name] = value
    return out


class _StageTimer:
    """HIP-event timing of named host stages (TIERKV_PROFILE=1): each
    ``end`` waits for the stage's GPU work, as the reference profiler does."""

    def __init__(self, enabled: bool):
        self.enabled = enabled
        self.totals: dict[str, float] = {}
        self.counts: dict[str, int] = {}

    def start(self):
        if not (self.enabled and torch.cuda.is_available()):
            return None
        mark = torch.cuda.Event(enable_timing=True)
        mark.record()
        return mark

    def end(self, name: str, mark) -> None:
        if mark is None:
            return
        done = torch.cuda.Event(enable_timing=True)
        done.record()
        done.synchronize()
        self.totals[name] = self.totals.get(name, 0.0) + float(mark.elapsed_time(done))
        self.counts[name] = self.counts.get(name, 0) + 1

    def summary(self) -> dict:
        return {name: (total, self.counts.get(name, 0), total / max(self.counts.get(name, 0), 1))
                for name, total in self.totals.items()}

    def clear(self) -> None:
        self.totals.clear()
        self.counts.clear()


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
        if prefill_scoring not in ("proxy", "attention"):
            raise ValueError('prefill_scoring must be "proxy" or "attention".')
        settings = _resolve_settings(dict(
            attention_backend=attention_backend, policy_interval=policy_interval, pool_chunk_blocks=pool_chunk_blocks,
            policy_on_new_block=policy_on_new_block, score_accumulation_mode=score_accumulation_mode,
            policy_mode=policy_mode, warm_budget=warm_budget, pool_layout=pool_layout))
        for name, value in settings.items():
            setattr(self, name, value)
        # Prefill block scores when the model's attention returns no
        # probabilities: "proxy" = the reference's sink + recency scores,
        # "attention" = the prefill block-score kernel (extension).
        self.prefill_scoring = prefill_scoring
        self.block_manager = block_manager
        self.num_layers = int(num_layers)
        self.block_size = int(block_size)
        self.hot_budget = int(hot_budget)
        self.max_seq_len = int(max_seq_len)
        self.max_blocks_per_layer = _ceil_div(self.max_seq_len, self.block_size)
        self.pool_blocks = self.num_layers * self.max_blocks_per_layer
        self.demoted_state = WARM_STATE
        self.cold_block_policy = "zero"
        self.tiered_layer_indices = set(range(self.num_layers))
        self.kv_pool = self._build_pool(warm_format)
        self.policy_engine = TierKVPolicyEngine(block_size=self.block_size, block_manager=block_manager)
        self._timer = _StageTimer(os.environ.get("TIERKV_PROFILE", "0") == "1")
        self.profile_enabled = self._timer.enabled
        self.profile_totals_ms = self._timer.totals
        self.profile_counts = self._timer.counts
        self.cache = TieredKVCache(self)
        self._restart()

    def _build_pool(self, warm_format: str):
        geometry = dict(num_layers=self.num_layers, block_size=self.block_size, max_seq_len=self.max_seq_len,
                        max_blocks_per_layer=self.max_blocks_per_layer, pool_blocks=self.pool_blocks,
                        pool_chunk_blocks=self.pool_chunk_blocks, warm_format=warm_format)
        if self.pool_layout == "dense":
            return TieredKVTensorPool(**geometry)
        hot, warm = self._compact_slot_capacities()
        return CompactTieredKVTensorPool(**geometry, max_hot_slots=self.num_layers * hot,
                                         max_warm_slots=self.num_layers * warm, hot_chunk_slots=max(1, hot),
                                         warm_chunk_slots=max(1, warm))

    def _compact_slot_capacities(self) -> tuple[int, int]:
        """Slots per layer of each compact tier (tierkv_policy.py:1628-1637):
        HOT holds the budget plus the blocks appended between two policy
        ticks and two spare; WARM the WARM budget plus two (or every block
        when nothing is evicted)."""
        if self.policy_mode == "hot_only":
            return self.max_blocks_per_layer, 0
        cap = self.max_blocks_per_layer
        hot = min(cap, max(2, self.hot_budget) + _ceil_div(self.policy_interval, self.block_size) + 2)
        warm = min(cap, self.warm_budget + 2) if self.policy_mode == "hot_warm_cold" else cap
        return max(1, hot), max(0, warm)

    def _restart(self) -> None:
        self.layer_states = {layer_idx: LayerRuntimeState() for layer_idx in range(self.num_layers)}
        self._step_cache: dict = {}   # layer -> the validated one-call decode launch (fused_decode_step)
        self.decode_step = 0
        self.current_query_length = 0
        self.policy_tick_this_forward = False

    # -- forward bracket -------------------------------------------------------
    def begin_forward(self, query_length: int) -> None:
        """A one-token forward is a decode step; every policy_interval-th
        decode step is a policy tick (tierkv_policy.py:1639-1644)."""
        self.current_query_length = int(query_length)
        decode = self.current_query_length == 1
        self.decode_step += int(decode)
        self.policy_tick_this_forward = decode and self.decode_step % self.policy_interval == 0

    def finish_forward(self) -> None:
        self.current_query_length = 0
        self.policy_tick_this_forward = False

    def reset(self, release_storage: bool = False) -> None:
        for seq_id in range(self.num_layers):
            self.block_manager.free_sequence(seq_id)
        (self.kv_pool.release if release_storage else self.kv_pool.clear)()
        self._restart()
        self._timer.clear()
        self.cache.reset()

    # -- profiling ------------------------------------------------------------
    def profile_start(self):
        return self._timer.start()

    def profile_end(self, name: str, start_event) -> None:
        self._timer.end(name, start_event)

    def profile_summary(self) -> dict[str, tuple[float, int, float]]:
        return self._timer.summary()

    def collect_memory_metrics(self) -> dict:
        return self.kv_pool.collect_memory_metrics(self.layer_states)

    # -- storing K/V ------------------------------------------------------------
    def _desired_prefill_states(self, num_blocks: int, block_scores: torch.Tensor) -> list[int]:
        """Initial tiers of a prompt's blocks (tierkv_policy.py:1695-1720),
        ranked by the label kernel."""
        n = int(num_blocks)
        if self.policy_mode == "hot_only" or n <= 2:
            return [HOT_STATE] * n
        if block_scores.ndim != 1 or len(block_scores) != n:
            raise ValueError("block_scores must be a 1D tensor matching prefill block count.")
        tiered = self.policy_mode == "hot_warm_cold"
        return _labels(block_scores, [HOT_STATE] * n, self.hot_budget, self.warm_budget if tiered else 0,
                       self.policy_mode, self.demoted_state)

    def _store_prompt_block(self, physical_idx: int, tier: int, src_k, src_v, start: int, length: int) -> None:
        pool = self.kv_pool
        if tier == HOT_STATE:
            pool._write_hot_range(physical_idx, 0, src_k, src_v, start, length)
        elif tier == WARM_STATE:
            pool._write_warm_range(physical_idx, src_k, src_v, start, length)
        elif tier == COLD_STATE:
            # A pool that holds nothing yet learns its geometry from the
            # block's tensors before recording it as evicted.
            if pool.is_allocated():
                pool.register_cold_block(physical_idx, length)
            else:
                pool._write_hot_range(physical_idx, 0, src_k, src_v, start, length)
                pool.demote_to_cold(physical_idx)
        else:
            raise ValueError(f"Unsupported desired state: {tier}")

    def append_prefill_with_policy(self, seq_id: int, key_states: torch.Tensor, value_states: torch.Tensor,
                                   block_scores: torch.Tensor) -> None:
        """Store a prompt with each block going straight to its tier
        (tierkv_policy.py:1722-1766): HOT copied, WARM quantized, COLD
        metadata only; one copy launch and one quantize launch for the whole
        prompt.  Decode tokens then start a new block."""
        if key_states.shape[-2] != value_states.shape[-2]:
            raise ValueError("Key and value states must have the same sequence length.")
        cursor = self.layer_states[seq_id]
        if cursor.num_blocks != 0 or cursor.open_physical_idx is not None:
            raise RuntimeError("append_prefill_with_policy expects an empty layer cache.")
        total = int(key_states.shape[-2])
        n = _ceil_div(total, self.block_size)
        if n > self.max_blocks_per_layer:
            raise RuntimeError(f"Layer {seq_id} exceeded max_blocks_per_layer={self.max_blocks_per_layer}.")
        tiers = self._desired_prefill_states(n, block_scores)
        pool = self.kv_pool
        src_k, src_v = pool._source(key_states, value_states)
        with pool._batch():
            for logical_idx, tier in enumerate(tiers):
                physical_idx = self.block_manager.allocate_block(seq_id)
                if tier != HOT_STATE:
                    self.block_manager.update_block_state(seq_id, logical_idx, tier)
                start = logical_idx * self.block_size
                self._store_prompt_block(pool._check_physical_idx(physical_idx), tier, src_k, src_v, start,
                                         min(self.block_size, total - start))
                pool.set_block_entry(seq_id, logical_idx, physical_idx, tier)
        cursor.num_blocks, cursor.open_physical_idx, cursor.open_token_count = n, None, 0

    def _placements(self, seq_id: int, cursor: LayerRuntimeState, tokens: int):
        """Where ``tokens`` appended tokens go: yields (physical block, its new
        logical index or None, position in the block, token count), opening
        a block from the BlockManager whenever none is open."""
        while tokens > 0:
            new_logical = None
            if cursor.open_physical_idx is None:
                cursor.open_physical_idx = self.block_manager.allocate_block(seq_id)
                cursor.open_token_count = 0
                new_logical = cursor.num_blocks
                if new_logical >= self.max_blocks_per_layer:
                    raise RuntimeError(f"Layer {seq_id} exceeded max_blocks_per_layer={self.max_blocks_per_layer}.")
                self.kv_pool._check_physical_idx(cursor.open_physical_idx)
            take = min(self.block_size - cursor.open_token_count, tokens)
            yield cursor.open_physical_idx, new_logical, cursor.open_token_count, take
            tokens -= take
            cursor.open_token_count += take
            if cursor.open_token_count == self.block_size:
                cursor.open_physical_idx, cursor.open_token_count = None, 0

    def append_to_layer(self, seq_id: int, key_states: torch.Tensor, value_states: torch.Tensor) -> bool:
        """Append tokens to a layer (tierkv_policy.py:1768-1816): the open
        block first, then new HOT blocks; a WARM open block is promoted
        before it takes tokens.  Returns whether a block was allocated."""
        if key_states.shape[-2] != value_states.shape[-2]:
            raise ValueError("Key and value states must have the same sequence length.")
        cursor = self.layer_states[seq_id]
        pool = self.kv_pool
        src_k, src_v = pool._source(key_states, value_states)
        p = cursor.open_physical_idx
        if p is not None and src_k.shape[-2] == 1 and pool.get_physical_state(p) == HOT_STATE:
            # A decode step's token into the open HOT block (an open block has
            # room: a full one is closed): the one write of the general path
            # below, without its placement loop.
            pool._append_token(p, cursor.open_token_count, src_k, src_v)
            cursor.open_token_count += 1
            if cursor.open_token_count == self.block_size:
                cursor.open_physical_idx, cursor.open_token_count = None, 0
            return False
        opened = False
        consumed = 0
        with pool._batch():
            for physical_idx, new_logical, position, take in self._placements(seq_id, cursor,
                                                                              int(key_states.shape[-2])):
                opened = opened or new_logical is not None
                if pool.get_physical_state(physical_idx) == WARM_STATE:
                    pool.promote_to_hot(physical_idx)
                pool._write_hot_range(physical_idx, position, src_k, src_v, consumed, take)
                consumed += take
                if new_logical is not None:
                    pool.set_block_entry(seq_id, new_logical, physical_idx, HOT_STATE)
                    cursor.num_blocks += 1
        return opened

    def append_tokens(self, layer_idx: int, key_states: torch.Tensor, value_states: torch.Tensor) -> bool:
        return self.append_to_layer(layer_idx, key_states, value_states)

    # -- reading K/V and tables -------------------------------------------------
    def reconstruct_layer(self, seq_id: int, allow_decode_reconstruct: bool = False):
        """Dense fp16 K/V of a layer in logical order (tierkv_policy.py:1818-1841)."""
        if self.attention_backend == "triton" and self.current_query_length == 1 and not allow_decode_reconstruct:
            raise RuntimeError("Decode reconstruction is disabled for the Triton TierKV hot path.")
        ids = self.block_manager.get_physical_indices(seq_id)
        states = self.block_manager.get_states(seq_id)
        if not ids:
            return None, None, ids, states
        parts = [self.kv_pool.get_dequantized_block(p, s) for p, s in zip(ids, states)]
        key = torch.cat([k for k, _ in parts], dim=-2).contiguous()
        value = torch.cat([v for _, v in parts], dim=-2).contiguous()
        return key, value, ids, states

    def sync_gpu_block_tables(self, seq_id: int) -> None:
        ids = self.block_manager.get_physical_indices(seq_id)
        self.kv_pool.sync_gpu_block_tables(seq_id, ids, self.block_manager.get_states(seq_id))
        self.layer_states[seq_id].num_blocks = len(ids)

    def sync_storage_states(self, seq_id: int) -> None:
        """Move every block of a layer to the tier the BlockManager now gives
        it (tierkv_policy.py:1849-1867), all in one batch: one demote launch,
        one promote launch, one table push."""
        pool = self.kv_pool
        pairs = zip(self.block_manager.get_physical_indices(seq_id), self.block_manager.get_states(seq_id))
        settled = pool._state_settled if pool.is_allocated() and pool._tables is not None else None
        with pool._batch():
            for logical_idx, (physical_idx, state) in enumerate(pairs):
                if settled is not None and settled(seq_id, logical_idx, physical_idx, state):
                    continue   # both calls below would do nothing
                pool.retier(physical_idx, state)
                pool.set_block_state(seq_id, logical_idx, state)

    def get_layer_table(self, seq_id: int):
        table, states = self.kv_pool.get_layer_table(seq_id)
        return table, states, self.kv_pool.get_layer_lengths(seq_id), self.layer_states[seq_id].num_blocks

    def fused_decode_step(self, seq_id: int, query_states, key_states, value_states, num_key_value_groups: int,
                          scaling: float):
        """The decode forward's append_to_layer, get_layer_table and
        tierkv_decode_attention (modeling_llama.py:419-456) as one C call,
        for the steps that are nothing else: one token into the layer's open
        HOT block or into a block it opens, no policy due and no scores
        collected.  Returns the attention output [1, 1, H, D], or None
        (nothing done) for any other step, which then takes the general
        path; both leave the same state."""
        if self._tiered(seq_id) and (self.policy_tick_this_forward or self.score_accumulation_mode == "every_step"):
            return None
        if (self._timer.enabled or _lib.env_flag("TIERKV_CHECK_ERRORS") or os.environ.get("TIERKV_FUSED_STEP") == "0"
                or not hasattr(self.kv_pool, "_decode_step")):
            return None
        cursor = self.layer_states[seq_id]
        p = cursor.open_physical_idx
        if key_states.shape[-2] != 1 or value_states.shape[-2] != 1:
            return None
        if p is None:
            # The token opens a block: placed as append_to_layer places it
            # (BlockManager id, HOT slot, table entry), unless the allocation
            # itself is due to run the policy.
            if self.policy_on_new_block and self._tiered(seq_id):
                return None
            if not self.kv_pool._fused_inputs_ok(query_states, key_states, value_states, 4):
                return None
            p = self._open_block(seq_id, cursor, key_states)
        out = self.kv_pool._decode_step(seq_id, p, cursor.open_token_count, cursor.num_blocks, query_states,
                                        key_states, value_states, num_key_value_groups, scaling, self._step_cache)
        if out is not None:
            cursor.open_token_count += 1
            if cursor.open_token_count == self.block_size:
                cursor.open_physical_idx, cursor.open_token_count = None, 0
        return out

    def _open_block(self, seq_id: int, cursor: LayerRuntimeState, key_states) -> int:
        """_placements' block opening and append_to_layer's placement of its
        first token, for a token the decode step's own launch writes: the
        BlockManager id, the HOT slot (the token counted), the table entry."""
        p = self.block_manager.allocate_block(seq_id)
        cursor.open_physical_idx, cursor.open_token_count = p, 0
        new_logical = cursor.num_blocks
        if new_logical >= self.max_blocks_per_layer:
            raise RuntimeError(f"Layer {seq_id} exceeded max_blocks_per_layer={self.max_blocks_per_layer}.")
        pool = self.kv_pool
        pool._check_physical_idx(p)
        pool._open_hot(p, key_states)
        pool.set_block_entry(seq_id, new_logical, p, HOT_STATE)
        cursor.num_blocks += 1
        return p

    # -- policy ---------------------------------------------------------------
    def _tiered(self, seq_id: int) -> bool:
        return seq_id in self.tiered_layer_indices and self.policy_mode != "hot_only"

    def should_run_decode_policy(self, seq_id: int, allocated_new_block: bool) -> bool:
        due = self.policy_tick_this_forward or (self.policy_on_new_block and allocated_new_block)
        return self._tiered(seq_id) and self.current_query_length == 1 and bool(due)

    def should_collect_decode_scores(self, seq_id: int, run_policy: bool) -> bool:
        return self._tiered(seq_id) and bool(run_policy or self.score_accumulation_mode == "every_step")

    def enforce_policy(self, seq_id: int, block_scores: torch.Tensor) -> None:
        if self.policy_mode == "hot_warm_cold":
            self.policy_engine.enforce_tiered_budget(seq_id, block_scores, self.hot_budget, self.warm_budget)
        elif self.policy_mode == "hot_warm":
            self.policy_engine.enforce_budget(seq_id, block_scores, self.hot_budget, demoted_state=self.demoted_state)

    def block_scores_from_probability_sums(self, seq_id: int, score_sums: torch.Tensor) -> torch.Tensor:
        """Per-block probability mass averaged over heads and divided by the
        block's token count (tierkv_policy.py:1905-1912), in the block-score
        kernel."""
        n = self.layer_states[seq_id].num_blocks
        if n == 0:
            return torch.empty(0, device=score_sums.device, dtype=torch.float32)
        _lib.require_gpu_tensor(score_sums, "score_sums")
        lengths = self.kv_pool.get_layer_lengths(seq_id)
        sums = score_sums.to(torch.float32).contiguous()
        out = torch.empty(n, dtype=torch.float32, device=sums.device)
        rc = _lib.lib().tierkv_block_scores_from_sums(_lib.ptr(sums), int(sums.shape[1]), _lib.ptr(lengths),
                                                     int(lengths.numel()), _lib.ptr(out), 1, int(sums.shape[0]), n,
                                                     _lib.stream_of(sums.device))
        _lib.check(rc, "tierkv_block_scores_from_sums")
        return out


# ---------------------------------------------------------------------------
# Module-level runtime handle (tierkv_policy.py:1915-2044).
# ---------------------------------------------------------------------------

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
    options = dict(locals())
    return TieredKVRuntime(**options)


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
    """Replace the process-wide runtime (releasing the previous one's storage)
    and return its HF cache."""
    global _GLOBAL_TIERKV_RUNTIME
    options = dict(locals())
    reset_global_tierkv()
    _GLOBAL_TIERKV_RUNTIME = create_tierkv_runtime(**options)
    return _GLOBAL_TIERKV_RUNTIME.cache


# Metrics that add up over runtimes; the ratios are recomputed from the sums
# (tierkv_policy.py:1985-2032).
_SUMMED_KEYS = _TOKEN_KEYS + _MB_KEYS[:6] + (
    "physical_hot_pool_mb", "physical_warm_pool_mb", "physical_warm_meta_mb", "physical_total_kv_mb",
    "active_pool_blocks", "allocated_pool_blocks", "pool_blocks", "hot_slots_used", "hot_slots_capacity",
    "warm_slots_used", "warm_slots_capacity")


def _ratio(num: float, den: float) -> float:
    return num / den if den > 0 else 0.0


def aggregate_memory_metrics(metrics_list) -> dict:
    present = [m for m in metrics_list if m]
    if not present:
        return TieredKVTensorPool().collect_memory_metrics({})
    out = {key: sum(m.get(key, 0) for m in present) for key in _SUMMED_KEYS}
    resident = float(out["logical_resident_mb"])
    dense = float(out["logical_dense_equivalent_mb"])
    out["logical_compression_ratio"] = _ratio(resident, dense)
    out["logical_compression_x"] = _ratio(dense, resident)
    out["pool_utilization"] = out["active_pool_blocks"] / max(float(out["allocated_pool_blocks"]), 1.0)
    out["capacity_utilization"] = out["allocated_pool_blocks"] / max(float(out["pool_blocks"]), 1.0)
    out["physical_compression_x"] = _ratio(dense, float(out["physical_total_kv_mb"]))
    return out


def reset_global_tierkv() -> None:
    global _GLOBAL_TIERKV_RUNTIME
    if _GLOBAL_TIERKV_RUNTIME is not None:
        _GLOBAL_TIERKV_RUNTIME.reset(release_storage=True)
    _GLOBAL_TIERKV_RUNTIME = None


def get_global_tierkv_runtime():
    return _GLOBAL_TIERKV_RUNTIME

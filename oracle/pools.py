"""Compact tiered pool restatement (oracle; test infrastructure only).

Follows CompactTieredKVTensorPool (tierkv_policy.py:701-1365) with NumPy
storage: separate HOT and WARM slot pools; LIFO free lists refilled
``range(new - 1, old - 1, -1)`` on growth so ``pop`` hands out the lowest new
slot first (tierkv_policy.py:849-895, 897-915); per-layer tables indexed by
logical block holding the state-specific slot (-1 for COLD), the state and
the length (``_set_metadata``, 917-926; ``set_block_entry``, 1012-1027).

Migrations:
* ``write_hot_tokens`` (934-967): a new physical block pops a HOT slot;
  the tail after the written tokens is zeroed.
* ``write_warm_block`` (969-1002): frees the current slot, pops a WARM slot,
  quantizes the tokens, zero-pads the tail (codes 0, scale 1, zero 0).
* ``demote_to_warm`` (1042-1068): pops a WARM slot, quantizes [:length] of
  the HOT slot, frees the HOT slot (tail of the warm slot left as is).
* ``demote_to_cold`` (1070-1085), ``promote_to_hot`` (1087-1115, fp16
  dequant), ``register_cold_block`` (1004-1014).

``warm_format`` selects the reference per-token uint8 codec or the
per-(block, head) int8 absmax codec (scales [slots, H_kv] fp32).
``demotion_plan`` gives the (hot slot, warm slot) pairs that a batch of
demotions in ascending logical order produces (sync_storage_states,
tierkv_policy.py:1849-1867).

Pinned against a trajectory recorded from the reference pool itself
(tests/golden/make_golden.py) and the reference's slot-transition test
(main.py:779-828).
"""

from __future__ import annotations

import numpy as np

from . import COLD_STATE, HOT_STATE, WARM_STATE
from .codec import dequantize_ref_u8, quantize_absmax_i8, quantize_ref_u8


class CompactPoolOracle:
    def __init__(self, num_layers, block_size, max_blocks_per_layer, kv_heads, head_dim,
                 max_hot_slots, max_warm_slots, hot_chunk_slots, warm_chunk_slots,
                 warm_format="ref_u8"):
        self.num_layers = num_layers
        self.block_size = block_size
        self.kv_heads = kv_heads
        self.head_dim = head_dim
        self.max_hot_slots = max_hot_slots
        self.max_warm_slots = max_warm_slots
        self.hot_chunk = max(1, hot_chunk_slots)
        self.warm_chunk = max(1, warm_chunk_slots)
        self.warm_format = warm_format
        shape = (num_layers, max_blocks_per_layer)
        self.slot_table = np.full(shape, -1, np.int32)
        self.phys_table = np.full(shape, -1, np.int32)
        self.state_table = np.full(shape, COLD_STATE, np.int32)
        self.len_table = np.zeros(shape, np.int32)
        self.hot_k = np.zeros((0, kv_heads, block_size, head_dim), np.float16)
        self.hot_v = self.hot_k.copy()
        wdt = np.uint8 if warm_format == "ref_u8" else np.int8
        self.warm_k = np.zeros((0, kv_heads, block_size, head_dim), wdt)
        self.warm_v = self.warm_k.copy()
        if warm_format == "ref_u8":
            self.k_scale = np.ones((0, kv_heads, block_size, 1), np.float16)
            self.v_scale = self.k_scale.copy()
            self.k_zero = np.zeros((0, kv_heads, block_size, 1), np.float16)
            self.v_zero = self.k_zero.copy()
        else:
            self.k_scale = np.zeros((0, kv_heads), np.float32)
            self.v_scale = self.k_scale.copy()
            self.k_zero = self.v_zero = None
        self.hot_free: list[int] = []
        self.warm_free: list[int] = []
        self.states: dict[int, int] = {}
        self.slots: dict[int, int] = {}
        self.lengths: dict[int, int] = {}
        self.locations: dict[int, tuple[int, int]] = {}

    # -- growth / slots (tierkv_policy.py:849-915) --------------------------
    def _grow(self, arr, new_cap, fill):
        out = np.full((new_cap,) + arr.shape[1:], fill, arr.dtype)
        out[: arr.shape[0]] = arr
        return out

    def _alloc_hot(self):
        if not self.hot_free:
            old = self.hot_k.shape[0]
            if old >= self.max_hot_slots:
                raise RuntimeError("No HOT slots available in compact TierKV pool.")
            new = min(self.max_hot_slots, old + self.hot_chunk)
            self.hot_k = self._grow(self.hot_k, new, 0)
            self.hot_v = self._grow(self.hot_v, new, 0)
            self.hot_free.extend(range(new - 1, old - 1, -1))
        return self.hot_free.pop()

    def _alloc_warm(self):
        if not self.warm_free:
            old = self.warm_k.shape[0]
            if old >= self.max_warm_slots:
                raise RuntimeError("No WARM slots available in compact TierKV pool.")
            new = min(self.max_warm_slots, old + self.warm_chunk)
            self.warm_k = self._grow(self.warm_k, new, 0)
            self.warm_v = self._grow(self.warm_v, new, 0)
            if self.warm_format == "ref_u8":
                self.k_scale = self._grow(self.k_scale, new, 1)
                self.v_scale = self._grow(self.v_scale, new, 1)
                self.k_zero = self._grow(self.k_zero, new, 0)
                self.v_zero = self._grow(self.v_zero, new, 0)
            else:
                self.k_scale = self._grow(self.k_scale, new, 0)
                self.v_scale = self._grow(self.v_scale, new, 0)
            self.warm_free.extend(range(new - 1, old - 1, -1))
        return self.warm_free.pop()

    def _set_metadata(self, phys, state, slot, length):
        self.states[phys] = state
        self.slots[phys] = slot
        self.lengths[phys] = length
        loc = self.locations.get(phys)
        if loc is not None:
            self.state_table[loc] = state
            self.slot_table[loc] = slot
            self.len_table[loc] = length

    def _quantize_into(self, slot, k, v, length, pad_tail):
        if self.warm_format == "ref_u8":
            for src, codes, scale, zero in ((k, self.warm_k, self.k_scale, self.k_zero),
                                            (v, self.warm_v, self.v_scale, self.v_zero)):
                q, s, z = quantize_ref_u8(src)
                codes[slot, :, :length] = q
                scale[slot, :, :length] = s
                zero[slot, :, :length] = z
                if pad_tail and length < self.block_size:
                    codes[slot, :, length:] = 0
                    scale[slot, :, length:] = 1
                    zero[slot, :, length:] = 0
        else:
            for src, codes, scale in ((k, self.warm_k, self.k_scale), (v, self.warm_v, self.v_scale)):
                q, s = quantize_absmax_i8(src)
                codes[slot, :, :length] = q
                codes[slot, :, length:] = 0
                scale[slot] = s

    # -- public API -----------------------------------------------------------
    def set_block_entry(self, layer, logical, phys, state):
        self.locations[phys] = (layer, logical)
        self.phys_table[layer, logical] = phys
        self.state_table[layer, logical] = state
        self.slot_table[layer, logical] = self.slots.get(phys, -1)
        self.len_table[layer, logical] = self.lengths.get(phys, 0)

    def write_hot_tokens(self, phys, start, k, v):
        tokens = k.shape[1]
        cur = self.states.get(phys)
        if cur == COLD_STATE:
            raise KeyError(f"Physical block {phys} is COLD and cannot be promoted.")
        if cur == WARM_STATE:
            self.promote_to_hot(phys)
        slot = self.slots.get(phys)
        if slot is None or cur is None:
            slot = self._alloc_hot()
        self.hot_k[slot, :, start:start + tokens] = k
        self.hot_v[slot, :, start:start + tokens] = v
        self.hot_k[slot, :, start + tokens:] = 0
        self.hot_v[slot, :, start + tokens:] = 0
        self._set_metadata(phys, HOT_STATE, slot, start + tokens)

    def write_warm_block(self, phys, k, v):
        length = k.shape[1]
        cur = self.states.get(phys)
        if cur == HOT_STATE:
            self.hot_free.append(self.slots[phys])
        elif cur == WARM_STATE:
            self.warm_free.append(self.slots[phys])
        elif cur == COLD_STATE:
            raise KeyError(f"Physical block {phys} is COLD and cannot be promoted.")
        slot = self._alloc_warm()
        self._quantize_into(slot, k, v, length, pad_tail=True)
        self._set_metadata(phys, WARM_STATE, slot, length)

    def register_cold_block(self, phys, length):
        st = self.states.get(phys)
        if st == HOT_STATE:
            self.hot_free.append(self.slots[phys])
        elif st == WARM_STATE:
            self.warm_free.append(self.slots[phys])
        self._set_metadata(phys, COLD_STATE, -1, int(length))

    def demote_to_warm(self, phys):
        st = self.states.get(phys)
        if st == WARM_STATE:
            return
        if st != HOT_STATE:
            raise KeyError(f"Physical block {phys} is not present in HOT storage.")
        length = self.lengths[phys]
        hot = self.slots[phys]
        warm = self._alloc_warm()
        self._quantize_into(warm, self.hot_k[hot, :, :length], self.hot_v[hot, :, :length], length, pad_tail=False)
        self.hot_free.append(hot)
        self._set_metadata(phys, WARM_STATE, warm, length)

    def demote_to_cold(self, phys):
        st = self.states.get(phys)
        if st == COLD_STATE:
            return
        if st == HOT_STATE:
            self.hot_free.append(self.slots[phys])
        elif st == WARM_STATE:
            self.warm_free.append(self.slots[phys])
        else:
            raise KeyError(f"Physical block {phys} is not present in HOT or WARM storage.")
        self._set_metadata(phys, COLD_STATE, -1, self.lengths.get(phys, 0))

    def promote_to_hot(self, phys):
        st = self.states.get(phys)
        if st == HOT_STATE:
            return
        if st != WARM_STATE:
            raise KeyError(f"Physical block {phys} is not eligible for HOT promotion.")
        length = self.lengths[phys]
        warm = self.slots[phys]
        hot = self._alloc_hot()
        if self.warm_format == "ref_u8":
            k = dequantize_ref_u8(self.warm_k[warm, :, :length], self.k_scale[warm, :, :length], self.k_zero[warm, :, :length])
            v = dequantize_ref_u8(self.warm_v[warm, :, :length], self.v_scale[warm, :, :length], self.v_zero[warm, :, :length])
        else:
            k = (self.warm_k[warm, :, :length].astype(np.float32) * self.k_scale[warm][:, None, None]).astype(np.float16)
            v = (self.warm_v[warm, :, :length].astype(np.float32) * self.v_scale[warm][:, None, None]).astype(np.float16)
        self.hot_k[hot, :, :length] = k
        self.hot_v[hot, :, :length] = v
        self.warm_free.append(warm)
        self._set_metadata(phys, HOT_STATE, hot, length)


def demotion_plan(warm_free, num_demotions, allocated_warm, max_warm, warm_chunk):
    """Warm slots that ``num_demotions`` successive ``_alloc_warm_slot`` calls
    return (tierkv_policy.py:871-905): pop from the LIFO free list, growing by
    ``warm_chunk`` when empty.  On a fresh pool this is 0, 1, 2, ..."""
    free = list(warm_free)
    cap = allocated_warm
    out = []
    for _ in range(num_demotions):
        if not free:
            if cap >= max_warm:
                raise RuntimeError("No WARM slots available in compact TierKV pool.")
            new = min(max_warm, cap + max(1, warm_chunk))
            free.extend(range(new - 1, cap - 1, -1))
            cap = new
        out.append(free.pop())
    return out, free, cap

"""CPU model of the batched tiered runtime (test infrastructure only).

Each sequence follows the reference runtime's rules (tierkv_policy.py):

* prefill tiers: _desired_prefill_states (1695-1720) on the given scores;
  HOT blocks copied with a zeroed tail (write_hot_tokens, 934-967), WARM
  blocks quantized with a padded tail (write_warm_block, 969-1002), COLD
  blocks metadata only (register_cold_block, 1004-1014);
* decode append: the open block first -- the last block, while an earlier
  append left it partially filled; a prefill leaves no open block
  (append_prefill_with_policy resets it, 1764-1766) -- then new HOT blocks
  (append_to_layer, 1768-1816);
* policy tick: block_scores_from_probability_sums (1905-1912), then
  enforce_budget / enforce_tiered_budget (1391-1477), then the storage moves
  of sync_storage_states (1849-1867): HOT->WARM quantizes the block's first
  `length` tokens into a new WARM slot (demote_to_warm, 1042-1068; the
  reference codec leaves the tail as it was), WARM->HOT dequantizes
  (promote_to_hot, 1087-1115), ->COLD frees the slot (demote_to_cold,
  1070-1085).

What the reference leaves open -- it serves one sequence with host free
lists -- is fixed here the way the device runtime fixes it: one pool pair
per layer shared by the batch, free-slot stacks popped from the top, and a
tick's slots reused within it in five steps, each in (sequence, block)
order: WARM->COLD slots pushed on the WARM stack, demotions popping it,
demoted and HOT->COLD slots pushed on the HOT stack, promotions popping it,
promoted blocks' WARM slots pushed last; a migration with no free slot is
left undone; the demotions' data moves before the promotions'.  The
scores' fp32 sum over heads is sequential (the device order); ATen's
order is not pinned.
"""

from __future__ import annotations

import numpy as np

from .codec import quantize_absmax_i8, quantize_ref_u8, dequantize_ref_u8
from .policy import block_mass_from_sums, desired_prefill_states, tier_labels

HOT, WARM, COLD = 0, 1, 2


class BatchedRuntimeOracle:
    def __init__(self, batch, kv_heads, head_dim, block_size, max_blocks, hot_slots, warm_slots,
                 policy_mode="hot_warm_cold", warm_format="absmax_i8"):
        self.B, self.kv, self.D, self.bs, self.maxb = batch, kv_heads, head_dim, block_size, max_blocks
        self.hot_slots, self.warm_slots = hot_slots, warm_slots
        self.mode = policy_mode
        self.fmt = warm_format
        self.table = np.full((batch, max_blocks), -1, np.int32)
        self.states = np.full((batch, max_blocks), COLD, np.int32)
        self.lengths = np.zeros((batch, max_blocks), np.int32)
        self.nb = np.zeros(batch, np.int32)
        self.open = np.zeros(batch, bool)
        self.hot_k = np.zeros((hot_slots, kv_heads, block_size, head_dim), np.float16)
        self.hot_v = np.zeros_like(self.hot_k)
        if warm_format == "absmax_i8":
            self.warm_k = np.zeros((warm_slots, kv_heads, block_size, head_dim), np.int8)
            self.k_scale = np.zeros((warm_slots, kv_heads), np.float32)
        else:
            self.warm_k = np.zeros((warm_slots, kv_heads, block_size, head_dim), np.uint8)
            self.k_scale = np.ones((warm_slots, kv_heads, block_size, 1), np.float16)
            self.k_zero = np.zeros((warm_slots, kv_heads, block_size, 1), np.float16)
            self.v_zero = np.zeros_like(self.k_zero)
        self.warm_v = np.zeros_like(self.warm_k)
        self.v_scale = np.zeros_like(self.k_scale) if warm_format == "absmax_i8" else np.ones_like(self.k_scale)
        self.hot_free: list[int] = []
        self.warm_free: list[int] = []
        self.migrations = {"demote": 0, "promote": 0, "evict": 0, "promote_into_freed": 0}

    # -- codec ---------------------------------------------------------------

    def _quantize_into(self, slot, k, v, length, pad_tail):
        """k, v fp16 [kv, length, D] into WARM slot `slot`."""
        for src, codes, scale, zero in ((k, self.warm_k, self.k_scale, getattr(self, "k_zero", None)),
                                        (v, self.warm_v, self.v_scale, getattr(self, "v_zero", None))):
            if self.fmt == "absmax_i8":
                q, s = quantize_absmax_i8(src[None].astype(np.float16))
                codes[slot, :, :length] = q[0]
                codes[slot, :, length:] = 0
                scale[slot] = np.asarray(s).reshape(self.kv)
            else:
                q, s, z = quantize_ref_u8(src[None].astype(np.float16))
                codes[slot, :, :length] = q[0]
                scale[slot, :, :length] = s[0]
                zero[slot, :, :length] = z[0]
                if pad_tail:
                    codes[slot, :, length:] = 0
                    scale[slot, :, length:] = 1
                    zero[slot, :, length:] = 0

    def _dequantize(self, slot, length):
        out = []
        for codes, scale, zero in ((self.warm_k, self.k_scale, getattr(self, "k_zero", None)),
                                   (self.warm_v, self.v_scale, getattr(self, "v_zero", None))):
            if self.fmt == "absmax_i8":
                x = (codes[slot, :, :length].astype(np.float32) * scale[slot][:, None, None]).astype(np.float16)
            else:
                x = dequantize_ref_u8(codes[slot, :, :length][None], scale[slot, :, :length][None],
                                      zero[slot, :, :length][None])[0]
            out.append(x)
        return out

    # -- runtime steps --------------------------------------------------------

    def prefill(self, k, v, scores_per_seq, hot_budget, warm_budget):
        """k, v fp16 [B, kv, T, D]."""
        B, kv, T, D = k.shape
        n = -(-T // self.bs)
        nh = nw = 0
        for b in range(B):
            tiers = desired_prefill_states(n, scores_per_seq[b], hot_budget, warm_budget, self.mode)
            for i, s in enumerate(tiers):
                ln = min(self.bs, T - i * self.bs)
                self.lengths[b, i] = ln
                self.states[b, i] = s
                blk_k = k[b, :, i * self.bs: i * self.bs + ln]
                blk_v = v[b, :, i * self.bs: i * self.bs + ln]
                if s == HOT:
                    self.table[b, i] = nh
                    self.hot_k[nh] = 0
                    self.hot_v[nh] = 0
                    self.hot_k[nh, :, :ln] = blk_k
                    self.hot_v[nh, :, :ln] = blk_v
                    nh += 1
                elif s == WARM:
                    self.table[b, i] = nw
                    self._quantize_into(nw, blk_k, blk_v, ln, pad_tail=True)
                    nw += 1
            self.nb[b] = n
            self.open[b] = False
        self.hot_free = list(range(self.hot_slots - 1, nh - 1, -1))
        self.warm_free = list(range(self.warm_slots - 1, nw - 1, -1))

    def append(self, k1, v1):
        """One token per sequence: k1, v1 fp16 [B, kv, 1, D]."""
        needs = []
        for b in range(self.B):
            n = int(self.nb[b])
            open_ = bool(self.open[b]) and n > 0 and self.states[b, n - 1] == HOT and self.lengths[b, n - 1] < self.bs
            needs.append(0 if open_ else 1)
        if sum(needs) > len(self.hot_free):
            raise RuntimeError("no free HOT slot")
        for b in range(self.B):
            n = int(self.nb[b])
            if needs[b]:
                slot = self.hot_free.pop()
                self.table[b, n] = slot
                self.states[b, n] = HOT
                self.lengths[b, n] = 1
                self.nb[b] = n + 1
                pos = 0
            else:
                slot = int(self.table[b, n - 1])
                pos = int(self.lengths[b, n - 1])
                self.lengths[b, n - 1] = pos + 1
            self.hot_k[slot, :, pos] = k1[b, :, 0]
            self.hot_v[slot, :, pos] = v1[b, :, 0]
            self.open[b] = self.lengths[b, int(self.nb[b]) - 1] < self.bs

    def tick(self, score_sums, hot_budget, warm_budget, scores=None):
        """score_sums fp32 [B, H, >= n]; every sequence has the same n.  Given
        ``scores`` [B, n], they replace the block mass of the sums."""
        n = int(self.nb.max())
        if scores is None:
            scores = block_mass_from_sums(score_sums, self.lengths, n)
        scores = np.asarray(scores, np.float32)
        want = tier_labels(scores, self.states[:, :n], hot_budget, warm_budget, mode=self.mode)
        want = np.where(self.states[:, :n] == COLD, COLD, want)
        cells = [(b, i) for b in range(self.B) for i in range(n)]
        cur = {c: int(self.states[c]) for c in cells}
        want_of = {c: int(want[c]) for c in cells}
        slot_of = {c: int(self.table[c]) for c in cells}
        dem = [c for c in cells if cur[c] == HOT and want_of[c] == WARM]
        pro = [c for c in cells if cur[c] == WARM and want_of[c] == HOT]
        # 1. WARM -> COLD slots go on the WARM stack (top = end of the list).
        self.warm_free += [slot_of[c] for c in cells if cur[c] == WARM and want_of[c] == COLD]
        # 2. Demotions pop the WARM stack.
        wtop = len(self.warm_free)
        ndem = min(len(dem), wtop)
        dem_slot = {dem[k]: self.warm_free[wtop - 1 - k] for k in range(ndem)}
        self.warm_free = self.warm_free[: wtop - ndem]
        # 3. Demoted and HOT -> COLD slots go on the HOT stack.
        hot_before = len(self.hot_free)
        self.hot_free += [slot_of[c] for c in cells
                          if c in dem_slot or (cur[c] == HOT and want_of[c] == COLD)]
        # 4. Promotions pop the HOT stack.
        htop = len(self.hot_free)
        npro = min(len(pro), htop)
        # promotions landing in a slot this tick freed (the stack's top)
        self.migrations["promote_into_freed"] += min(npro, htop - hot_before)
        pro_slot = {pro[k]: self.hot_free[htop - 1 - k] for k in range(npro)}
        self.hot_free = self.hot_free[: htop - npro]
        # 5. Promoted blocks' WARM slots go on the WARM stack.
        self.warm_free += [slot_of[c] for c in pro[:npro]]
        moves_dem, moves_pro = [], []
        for c in cells:
            ln = int(self.lengths[c])
            if c in dem_slot:
                moves_dem.append((slot_of[c], dem_slot[c], ln))
                self.table[c] = dem_slot[c]
                self.states[c] = WARM
            elif c in pro_slot:
                moves_pro.append((slot_of[c], pro_slot[c], ln))
                self.table[c] = pro_slot[c]
                self.states[c] = HOT
            elif want_of[c] == COLD and cur[c] != COLD:
                self.migrations["evict"] += 1
                self.table[c] = -1
                self.states[c] = COLD
        self.migrations["demote"] += ndem
        self.migrations["promote"] += npro
        # Data movement: every demotion reads its HOT slot before any
        # promotion writes one (a promotion may land in a slot a demotion
        # freed); no demotion lands in a slot a promotion reads.
        for src, dst, ln in moves_dem:
            self._quantize_into(dst, self.hot_k[src, :, :ln], self.hot_v[src, :, :ln], ln, pad_tail=False)
        for src, dst, ln in moves_pro:
            k, v = self._dequantize(src, ln)
            self.hot_k[dst, :, :ln] = k
            self.hot_v[dst, :, :ln] = v
        return scores, want

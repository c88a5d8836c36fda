"""Batched tiered KV-cache runtime on MI355X.

The reference's ``TieredKVRuntime`` (tierkv_policy.py:1534-1912) serves one
sequence: its tables are per layer, its slots come from host free lists, and
every policy tick reads scores back to the host candidate by candidate
(1424, 1462).  This runtime keeps the same per-sequence semantics for a batch
of B sequences advancing in lockstep, with everything a decode step touches
resident on the device:

* per layer, compact pools (HOT fp16, WARM int8 absmax or the reference's
  uint8 + fp16 scale/zero), ``[B, max_blocks]`` slot / state / length tables,
  per-sequence block counts, and free-slot stacks;
* ``prefill`` writes each sequence's prompt blocks straight into the tier the
  policy gives them (HOT copy, WARM quantize, COLD metadata only) --
  ``append_prefill_with_policy`` (1722-1766) without an fp16 detour for WARM
  blocks;
* ``decode_layer`` appends the step's K/V (``tierkv_runtime_append``: new HOT
  blocks popped on the device), runs the tiered decode kernel, and on policy
  steps runs ``tierkv_runtime_tick`` (scores -> labels -> migrations on the
  device).  The host never waits for the device inside a step.

Budgets are fractions of each sequence's current block count (BASELINE's
C5: 15 % HOT, 55 % WARM, the rest evicted), evaluated on the host from the
lockstep block count.
"""

from __future__ import annotations

import os

from dataclasses import dataclass

import torch

from . import _lib, kernels
from .tierkv_hip import DecodeWorkspace, tierkv_decode_attention

HOT_STATE, WARM_STATE, COLD_STATE = 0, 1, 2
_MODES = {"hot_warm": 1, "hot_warm_cold": 2}
ERROR_BITS = {1: "no free HOT slot", 2: "no free WARM slot", 4: "a table row is full",
              8: "a sequence's last block was not HOT"}


def _ceil_div(a: int, b: int) -> int:
    return (int(a) + int(b) - 1) // int(b)


def budget_blocks(fraction: float, num_blocks: int) -> int:
    """Blocks a tier may hold: round(fraction * num_blocks), half to even."""
    return int(round(float(fraction) * int(num_blocks)))


def prefill_states(num_blocks: int, scores, hot_budget: int, warm_budget: int, policy_mode: str) -> list[int]:
    """Initial tiers of a prompt's blocks (_desired_prefill_states,
    tierkv_policy.py:1695-1720): reserved HOT {0, n-1}, candidates ranked by
    score descending (ties to the lower index), top hot_budget-2 HOT, then
    warm_budget WARM (hot_warm_cold) or every other block WARM (hot_warm)."""
    n = int(num_blocks)
    if n <= 2:
        return [HOT_STATE] * n
    cand = [i for i in range(n) if i not in (0, n - 1)]
    order = sorted(cand, key=lambda i: float(scores[i]), reverse=True)
    extra = max(int(hot_budget) - 2, 0)
    hot = set(order[:extra])
    warm = set(order[extra: extra + max(int(warm_budget), 0)])
    out = []
    for i in range(n):
        if i in (0, n - 1) or i in hot:
            out.append(HOT_STATE)
        elif policy_mode == "hot_warm_cold":
            out.append(WARM_STATE if i in warm else COLD_STATE)
        else:
            out.append(WARM_STATE)
    return out


def recency_scores(num_blocks: int) -> list[float]:
    """Sink + recency proxy for prompts whose attention probabilities are not
    materialised (compute_prefill_block_scores, modeling_llama.py:280-302)."""
    n = int(num_blocks)
    if n <= 0:
        return []
    s = [float(i) / float(n - 1) if n > 1 else 0.0 for i in range(n)]
    s[0] = 1.0
    s[-1] = 1.0
    return s


def _strided_f16(t: torch.Tensor) -> torch.Tensor:
    """fp16 tensor whose head dimension is contiguous, with strides that are
    multiples of 8 elements and a 16-byte aligned start (copied otherwise)."""
    if t.dtype != torch.float16:
        raise ValueError("the fused rotary append takes fp16 tensors.")
    if t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:-1]) or t.data_ptr() % 16:
        t = t.contiguous()
    return t


@dataclass
class LayerStorage:
    hot_k: torch.Tensor
    hot_v: torch.Tensor
    warm_k: torch.Tensor
    warm_v: torch.Tensor
    k_scale: torch.Tensor
    k_zero: torch.Tensor | None
    v_scale: torch.Tensor
    v_zero: torch.Tensor | None
    table: torch.Tensor       # [B, max_blocks] slot (state-specific pool), -1 for COLD
    states: torch.Tensor      # [B, max_blocks]
    lengths: torch.Tensor     # [B, max_blocks]
    nblocks: torch.Tensor     # [B]
    open: torch.Tensor        # [B] 1 while the last block takes further appended tokens
    hot_free: torch.Tensor    # [hot capacity] free-slot stack
    warm_free: torch.Tensor   # [warm capacity]
    ctl: torch.Tensor         # [4] hot_top, warm_top, error bits, last append applied


class BatchedTieredKVRuntime:
    """Tiered KV cache for ``batch`` sequences of a ``num_layers`` model.

    ``cache`` is the HF cache object the model hooks (hf_llama) recognise;
    ``begin_forward`` / ``finish_forward`` follow the reference runtime's
    (tierkv_policy.py:1639-1648): a one-token forward is a decode step, and
    every ``policy_interval``-th decode step is a policy step."""

    is_batched = True

    def __init__(self, num_layers: int, batch: int, kv_heads: int, head_dim: int, max_seq_len: int,
                 block_size: int = 16, hot_fraction: float = 0.15, warm_fraction: float = 0.55,
                 policy_mode: str = "hot_warm_cold", policy_interval: int = 64,
                 warm_format: str = "absmax_i8", cold_mode: str = "masked", device=None,
                 prefill_scoring: str = "proxy", deterministic: bool | None = None):
        if policy_mode not in _MODES:
            raise ValueError('policy_mode must be "hot_warm" or "hot_warm_cold".')
        if warm_format not in kernels.WARM_FORMATS:
            raise ValueError('warm_format must be "absmax_i8" or "ref_u8".')
        if policy_interval <= 0:
            raise ValueError("policy_interval must be positive.")
        if prefill_scoring not in ("proxy", "attention"):
            raise ValueError('prefill_scoring must be "proxy" or "attention".')
        if not (0.0 <= hot_fraction <= 1.0 and 0.0 <= warm_fraction <= 1.0):
            raise ValueError("tier fractions must lie in [0, 1].")
        self.device = torch.device(device or "cuda")
        if self.device.type != "cuda":
            raise ValueError("the batched runtime needs a GPU (HIP) device.")
        _lib.lib()   # RuntimeError if the HIP library is not built
        self.num_layers = int(num_layers)
        self.batch = int(batch)
        self.kv_heads = int(kv_heads)
        self.head_dim = int(head_dim)
        self.block_size = int(block_size)
        self.max_seq_len = int(max_seq_len)
        self.max_blocks = _ceil_div(max_seq_len, block_size)
        self.hot_fraction = float(hot_fraction)
        self.warm_fraction = float(warm_fraction)
        self.policy_mode = policy_mode
        self.policy_interval = int(policy_interval)
        self.warm_format = warm_format
        self.cold_mode = cold_mode
        # Prefill block scores when the model's attention returns no
        # probabilities: "proxy" = sink + recency (the reference under SDPA),
        # "attention" = the prefill block-score kernel.
        self.prefill_scoring = prefill_scoring
        # Decode launches with a fixed tile share per wave: every step's
        # attention output is the same bits on every run (about 1-3 % of the
        # decode kernel's time, a few microseconds of a model step).  On by
        # default; TIERKV_DETERMINISTIC, when set, decides instead.
        if deterministic is None:
            env = os.environ.get("TIERKV_DETERMINISTIC")
            deterministic = True if env is None else env not in ("", "0")
        self.deterministic = bool(deterministic)
        n = self.max_blocks
        # Capacities per sequence, from the budgets: a tick reuses the slots it
        # frees (demotions take evicted WARM slots, promotions the HOT slots
        # that demotions free), so HOT holds at most its budget plus the
        # blocks appended between ticks, and WARM its budget plus a tick's
        # promotions (blocks still WARM until the promotion has read them).
        hot_max = max(2, budget_blocks(self.hot_fraction, n))
        appended = _ceil_div(self.policy_interval, self.block_size) + 2
        self.hot_per_seq = min(n, hot_max + appended)
        if policy_mode == "hot_warm":
            self.warm_per_seq = n
        else:
            self.warm_per_seq = min(n, budget_blocks(self.warm_fraction, n) + hot_max + 2)
        self.hot_slots = self.batch * self.hot_per_seq
        self.warm_slots = max(1, self.batch * self.warm_per_seq)
        self.layers = [self._new_layer() for _ in range(self.num_layers)]
        # Host copy of the (lockstep) block count and open-block fill per layer,
        # so launch sizes and budgets need no device read-back.
        self._blocks = [0] * self.num_layers
        self._open_tokens = [0] * self.num_layers
        self.seq_len = 0              # tokens per sequence (lockstep)
        self.decode_step = 0
        self.max_demotions = self.batch * self.hot_per_seq
        self.max_promotions = self.batch * self.hot_per_seq
        nbytes = _lib.lib().tierkv_runtime_tick_scratch_bytes(self.batch, self.max_blocks, self.max_demotions,
                                                              self.max_promotions)
        self.tick_scratch = torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device=self.device)
        self.current_query_length = 0
        self.policy_tick_this_forward = False
        self.fixed_launch_bound = False
        # The decode kernel's scratch: owned by the runtime, sized once for the
        # largest launch (max_blocks, with score sums) and never replaced, so
        # captured decode steps always replay on live memory.  Every launch of
        # the runtime is ordered on the caller's stream, so one serves all
        # layers.
        self.decode_workspace: DecodeWorkspace | None = None
        self._workspace_heads = 0
        # HF hooks: rotate q / k inside the decode append (fp16 models).
        self.fused_rope = True
        from .tierkv_policy import TieredKVCache
        self.cache = TieredKVCache(self)

    # -- storage ------------------------------------------------------------

    def _new_layer(self) -> LayerStorage:
        dev, kv, bs, d = self.device, self.kv_heads, self.block_size, self.head_dim
        hot = (self.hot_slots, kv, bs, d)
        warm = (self.warm_slots, kv, bs, d)
        if self.warm_format == "absmax_i8":
            wk = torch.zeros(warm, dtype=torch.int8, device=dev)
            wv = torch.zeros(warm, dtype=torch.int8, device=dev)
            ks = torch.zeros((self.warm_slots, kv), dtype=torch.float32, device=dev)
            vs = torch.zeros((self.warm_slots, kv), dtype=torch.float32, device=dev)
            kz = vz = None
        else:
            wk = torch.zeros(warm, dtype=torch.uint8, device=dev)
            wv = torch.zeros(warm, dtype=torch.uint8, device=dev)
            ks = torch.ones((self.warm_slots, kv, bs, 1), dtype=torch.float16, device=dev)
            vs = torch.ones((self.warm_slots, kv, bs, 1), dtype=torch.float16, device=dev)
            kz = torch.zeros((self.warm_slots, kv, bs, 1), dtype=torch.float16, device=dev)
            vz = torch.zeros((self.warm_slots, kv, bs, 1), dtype=torch.float16, device=dev)
        tab = (self.batch, self.max_blocks)
        return LayerStorage(
            hot_k=torch.zeros(hot, dtype=torch.float16, device=dev),
            hot_v=torch.zeros(hot, dtype=torch.float16, device=dev),
            warm_k=wk, warm_v=wv, k_scale=ks, k_zero=kz, v_scale=vs, v_zero=vz,
            table=torch.full(tab, -1, dtype=torch.int32, device=dev),
            states=torch.full(tab, COLD_STATE, dtype=torch.int32, device=dev),
            lengths=torch.zeros(tab, dtype=torch.int32, device=dev),
            nblocks=torch.zeros(self.batch, dtype=torch.int32, device=dev),
            open=torch.zeros(self.batch, dtype=torch.int32, device=dev),
            hot_free=torch.zeros(self.hot_slots, dtype=torch.int32, device=dev),
            warm_free=torch.zeros(self.warm_slots, dtype=torch.int32, device=dev),
            ctl=torch.zeros(4, dtype=torch.int32, device=dev))

    def budgets(self, num_blocks: int) -> tuple[int, int]:
        hot = max(2, budget_blocks(self.hot_fraction, num_blocks))
        warm = budget_blocks(self.warm_fraction, num_blocks)
        return hot, warm

    # -- prefill ------------------------------------------------------------

    def prefill_layer(self, layer: int, key_states: torch.Tensor, value_states: torch.Tensor,
                      block_scores=None) -> None:
        """Store a layer's prompt K/V [B, kv_heads, T, D] (the same T for every
        sequence) in its initial tiers.  block_scores: None (sink + recency
        proxy), a 1-D sequence shared by all sequences, or [B, n] per sequence."""
        st = self.layers[layer]
        if key_states.shape != value_states.shape or key_states.ndim != 4:
            raise ValueError("prefill K/V must be [batch, kv_heads, tokens, head_dim].")
        B, kv, T, d = (int(x) for x in key_states.shape)
        if (B, kv, d) != (self.batch, self.kv_heads, self.head_dim):
            raise ValueError("prefill K/V geometry does not match the runtime.")
        n = _ceil_div(T, self.block_size)
        if n > self.max_blocks:
            raise RuntimeError(f"prompt of {T} tokens exceeds max_seq_len={self.max_seq_len}.")
        k = key_states.to(torch.float16).contiguous()
        v = value_states.to(torch.float16).contiguous()
        hot_b, warm_b = self.budgets(n)
        if block_scores is None:
            per_seq = [recency_scores(n)] * B
        else:
            sc = torch.as_tensor(block_scores, dtype=torch.float32).cpu()
            per_seq = [sc.tolist()] * B if sc.ndim == 1 else [sc[b].tolist() for b in range(B)]
        bs = self.block_size
        table = torch.full((B, self.max_blocks), -1, dtype=torch.int32)
        states = torch.full((B, self.max_blocks), COLD_STATE, dtype=torch.int32)
        lengths = torch.zeros((B, self.max_blocks), dtype=torch.int32)
        hot_jobs, warm_jobs = [], []
        next_hot = next_warm = 0
        for b in range(B):
            tiers = prefill_states(n, per_seq[b], hot_b, warm_b, self.policy_mode)
            for i, s in enumerate(tiers):
                ln = min(bs, T - i * bs)
                lengths[b, i] = ln
                states[b, i] = s
                if s == HOT_STATE:
                    table[b, i] = next_hot
                    hot_jobs.append((b, i * bs, ln, next_hot))
                    next_hot += 1
                elif s == WARM_STATE:
                    table[b, i] = next_warm
                    warm_jobs.append((b, i * bs, ln, next_warm))
                    next_warm += 1
        if next_hot > self.hot_slots or next_warm > self.warm_slots:
            raise RuntimeError("prefill needs more slots than the runtime's pools hold.")
        dev = self.device
        if hot_jobs:
            self._write_hot(k, v, hot_jobs, st.hot_k, st.hot_v)
        if warm_jobs:
            # WARM blocks: fp16 tiles staged once, quantized into their slots.
            stage_k = torch.zeros((len(warm_jobs), kv, bs, d), dtype=torch.float16, device=dev)
            stage_v = torch.zeros_like(stage_k)
            self._write_hot(k, v, [(b, t0, ln, j) for j, (b, t0, ln, _) in enumerate(warm_jobs)], stage_k, stage_v)
            kernels.demote_to_warm(stage_k, stage_v, list(range(len(warm_jobs))), [w[3] for w in warm_jobs],
                                   [w[2] for w in warm_jobs], st.warm_k, st.warm_v, st.k_scale, st.k_zero,
                                   st.v_scale, st.v_zero, warm_format=self.warm_format, pad_tail=True)
        st.table.copy_(table)
        st.states.copy_(states)
        st.lengths.copy_(lengths)
        st.nblocks.fill_(n)
        st.open.zero_()      # decode tokens start a new block (tierkv_policy.py:1764-1766)
        self._blocks[layer] = n
        self._open_tokens[layer] = 0
        # Free stacks: popping from the top yields the lowest free slot first.
        st.hot_free[: self.hot_slots - next_hot].copy_(
            torch.arange(self.hot_slots - 1, next_hot - 1, -1, dtype=torch.int32))
        st.warm_free[: self.warm_slots - next_warm].copy_(
            torch.arange(self.warm_slots - 1, next_warm - 1, -1, dtype=torch.int32))
        st.ctl.copy_(torch.tensor([self.hot_slots - next_hot, self.warm_slots - next_warm, 0, 0],
                                  dtype=torch.int32))
        if layer == self.num_layers - 1:
            self.seq_len = T

    def _write_hot(self, k, v, jobs, dst_k, dst_v) -> None:
        lib = _lib.lib()
        cols = list(zip(*jobs))
        dev = self.device
        arr = [torch.tensor(c, dtype=torch.int32, device=dev) for c in cols]
        src_seq, src_tok, count, slot = arr
        zeros = torch.zeros_like(slot)
        rc = lib.tierkv_write_hot_tokens(
            _lib.ptr(k), _lib.ptr(v), int(k.shape[0]), int(k.shape[2]),
            _lib.ptr(src_seq), _lib.ptr(src_tok), _lib.ptr(count), _lib.ptr(slot), _lib.ptr(zeros),
            len(jobs), 1, _lib.ptr(dst_k), _lib.ptr(dst_v), int(dst_k.shape[0]),
            self.kv_heads, self.block_size, self.head_dim, _lib.stream_of(dev))
        _lib.check(rc, "tierkv_write_hot_tokens")

    # -- decode -------------------------------------------------------------

    def reserve_decode_workspace(self, num_heads: int) -> DecodeWorkspace:
        """Allocate (once) the fixed decode workspace for ``num_heads`` query
        heads; call it before capturing decode steps."""
        num_heads = int(num_heads)
        ws = self.decode_workspace
        if ws is None or self._workspace_heads != num_heads:
            if ws is not None and torch.cuda.is_current_stream_capturing():
                raise RuntimeError("the decode workspace cannot be replaced during HIP graph capture.")
            ws = DecodeWorkspace.for_shape(self.device, self.batch, num_heads, self.kv_heads, self.max_blocks,
                                           self.head_dim, block_size=self.block_size, return_scores=True)
            self.decode_workspace = ws
            self._workspace_heads = num_heads
        return ws

    def _advance_blocks(self, layer: int, tokens: int) -> int:
        """Mirror of the device append's block accounting (every sequence of
        the batch appends the same count): returns the new block count."""
        room = self.block_size - self._open_tokens[layer] if self._open_tokens[layer] else 0
        take = min(room, tokens)
        rest = tokens - take
        if rest > 0:
            self._blocks[layer] += _ceil_div(rest, self.block_size)
            last = rest - (_ceil_div(rest, self.block_size) - 1) * self.block_size
        else:
            last = self._open_tokens[layer] + take
        self._open_tokens[layer] = last if last < self.block_size else 0
        return self._blocks[layer]

    def begin_forward(self, query_length: int) -> None:
        self.current_query_length = int(query_length)
        self.policy_tick_this_forward = self.begin_step() if self.current_query_length == 1 else False

    def finish_forward(self) -> None:
        if self.current_query_length == 1:
            self.end_step()
        self.current_query_length = 0
        self.policy_tick_this_forward = False

    def begin_step(self) -> bool:
        """Start a decode step; returns whether it is a policy step (every
        policy_interval generated tokens, as begin_forward does at
        tierkv_policy.py:1639-1644)."""
        self.decode_step += 1
        return (self.decode_step % self.policy_interval) == 0

    def end_step(self) -> None:
        self.seq_len += 1

    def decode_layer(self, layer: int, query_states: torch.Tensor, key_states: torch.Tensor,
                     value_states: torch.Tensor, num_key_value_groups: int, scaling: float,
                     policy_step: bool = False, rope=None) -> torch.Tensor:
        """One decode step of one layer: append K/V [B, kv_heads, 1, D], attend
        with query [B, H, 1, D], and on policy steps re-tier the layer.  Returns
        the attention output [B, 1, H, D].

        rope: None (q and k already rotated), or the step's (cos, sin)
        [Bc, tokens, D] fp16 -- then q and k are the unrotated projections and
        the append kernel applies the rotation (transformers' fp16 op order)
        while copying K and producing the rotated q."""
        st = self.layers[layer]
        lib = _lib.lib()
        dev = self.device
        stream = _lib.stream_of(dev)
        tokens = int(key_states.shape[2])
        # blocks_hint: the lockstep block count before this append (none for
        # captured steps, whose arguments are fixed at capture).
        hint = 0 if self.fixed_launch_bound else self._blocks[layer]
        table_args = (_lib.ptr(st.table), _lib.ptr(st.states), _lib.ptr(st.lengths), self.max_blocks,
                      _lib.ptr(st.nblocks), _lib.ptr(st.open), self.batch, hint,
                      _lib.ptr(st.hot_k), _lib.ptr(st.hot_v), self.hot_slots, _lib.ptr(st.hot_free),
                      _lib.ptr(st.ctl), self.kv_heads, self.block_size, self.head_dim, stream)
        if rope is not None:
            cos, sin = rope
            q, k, v = (_strided_f16(t) for t in (query_states, key_states, value_states))
            cos, sin = (_strided_f16(t) for t in (cos, sin))
            if cos.shape != sin.shape or cos.stride() != sin.stride():
                raise ValueError("cos and sin must share shape and layout.")
            q_rot = torch.empty((self.batch, q.shape[1], tokens, self.head_dim), dtype=torch.float16, device=dev)
            cs_b = 0 if cos.shape[0] == 1 else cos.stride(0)
            rc = lib.tierkv_runtime_append_rope(
                _lib.ptr(q), q.stride(0), q.stride(1), q.stride(2), int(q.shape[1]), _lib.ptr(q_rot),
                _lib.ptr(k), k.stride(0), k.stride(1), k.stride(2),
                _lib.ptr(v), v.stride(0), v.stride(1), v.stride(2),
                _lib.ptr(cos), _lib.ptr(sin), cs_b, cos.stride(1), tokens, *table_args)
            _lib.check(rc, "tierkv_runtime_append_rope")
            query_states = q_rot
        else:
            k = key_states.to(torch.float16).contiguous()
            v = value_states.to(torch.float16).contiguous()
            rc = lib.tierkv_runtime_append(_lib.ptr(k), _lib.ptr(v), tokens, *table_args)
            _lib.check(rc, "tierkv_runtime_append")
        num_blocks = min(self._advance_blocks(layer, tokens), self.max_blocks)
        # With a fixed launch bound (captured decode steps) the kernel scans the
        # whole table row and takes each sequence's block count from nblocks on
        # the device, so the launch is the same at every step.
        bound = self.max_blocks if self.fixed_launch_bound else num_blocks
        out, sums = tierkv_decode_attention(
            query_states, st.table, st.states, st.lengths, st.hot_k, st.hot_v, st.warm_k, st.warm_v,
            st.k_scale, st.k_zero, st.v_scale, st.v_zero, bound, num_key_value_groups, scaling,
            return_scores=policy_step, cold_mode=self.cold_mode, seq_num_blocks=st.nblocks,
            workspace=self.reserve_decode_workspace(query_states.shape[1]), deterministic=self.deterministic)
        if policy_step:
            self.last_score_sums = sums   # the probability sums the tick ranked (kept for inspection)
            self.tick_layer(layer, sums, num_blocks)
        return out

    def tick_layer(self, layer: int, score_sums: torch.Tensor, num_blocks: int) -> None:
        st = self.layers[layer]
        lib = _lib.lib()
        hot_b, warm_b = self.budgets(num_blocks)
        rc = lib.tierkv_runtime_tick(
            _lib.ptr(score_sums), int(score_sums.shape[-1]), int(score_sums.shape[1]),
            _lib.ptr(st.table), _lib.ptr(st.states), _lib.ptr(st.lengths), self.max_blocks,
            _lib.ptr(st.nblocks), self.batch, hot_b, warm_b, _MODES[self.policy_mode],
            _lib.ptr(st.hot_k), _lib.ptr(st.hot_v), self.hot_slots, _lib.ptr(st.hot_free),
            _lib.ptr(st.warm_k), _lib.ptr(st.warm_v), self.warm_slots, _lib.ptr(st.warm_free),
            _lib.ptr(st.k_scale), _lib.ptr(st.k_zero), _lib.ptr(st.v_scale), _lib.ptr(st.v_zero),
            kernels.WARM_FORMATS[self.warm_format],
            _lib.ptr(st.ctl), _lib.ptr(self.tick_scratch), int(self.tick_scratch.numel()),
            self.max_demotions, self.max_promotions,
            self.kv_heads, self.block_size, self.head_dim, _lib.stream_of(self.device))
        _lib.check(rc, "tierkv_runtime_tick")

    # -- state and telemetry -------------------------------------------------

    def check_errors(self) -> None:
        """Raise RuntimeError if any layer's allocator flagged an error
        (synchronises)."""
        bits = 0
        for st in self.layers:
            bits |= int(st.ctl[2].item())
        if bits:
            msgs = [m for b, m in ERROR_BITS.items() if bits & b]
            raise RuntimeError("tiered KV runtime: " + "; ".join(msgs))

    def tier_counters(self, out: torch.Tensor | None = None) -> torch.Tensor:
        """Device int64 [6] = {HOT, WARM, COLD blocks, HOT, WARM, COLD tokens}
        summed over layers and sequences, computed on the device
        (``tierkv_tier_counts``) without a host sync; ``out`` is zeroed and
        reused when given."""
        lib = _lib.lib()
        if out is None:
            out = torch.zeros(6, dtype=torch.int64, device=self.device)
        else:
            out.zero_()
        stream = _lib.stream_of(self.device)
        for st in self.layers:
            rc = lib.tierkv_tier_counts(_lib.ptr(st.states), _lib.ptr(st.lengths), self.max_blocks,
                                        _lib.ptr(st.nblocks), self.batch, _lib.ptr(out), stream)
            _lib.check(rc, "tierkv_tier_counts")
        return out

    def memory_metrics(self) -> dict:
        """Resident KV bytes and tier counts over all layers and sequences
        (collect_memory_metrics, tierkv_policy.py:1193-1317) from the device
        counters: one host sync, for the single read-back."""
        kv, d = self.kv_heads, self.head_dim
        hot_blocks, warm_blocks, cold_blocks, hot_tok, warm_tok, cold_tok = (
            int(x) for x in self.tier_counters().cpu().tolist())
        fp16_tok = kv * d * 2 * 2
        int8_tok = kv * d * 2
        meta_tok = kv * 4 * 2 if self.warm_format == "ref_u8" else 0
        meta_block = kv * 4 * 2 if self.warm_format == "absmax_i8" else 0
        resident = hot_tok * fp16_tok + warm_tok * (int8_tok + meta_tok) + warm_blocks * meta_block
        dense = (hot_tok + warm_tok + cold_tok) * fp16_tok
        physical = 0
        for st in self.layers:
            for t in (st.hot_k, st.hot_v, st.warm_k, st.warm_v, st.k_scale, st.k_zero, st.v_scale, st.v_zero):
                if t is not None:
                    physical += t.numel() * t.element_size()
        return {
            "hot_blocks": hot_blocks, "warm_blocks": warm_blocks, "cold_blocks": cold_blocks,
            "hot_tokens": hot_tok, "warm_tokens": warm_tok, "cold_tokens": cold_tok,
            "resident_kv_bytes": resident, "dense_equivalent_bytes": dense,
            "compression_x": dense / resident if resident else 0.0,
            # HBM the pools hold (what the runtime allocates, free slots
            # included) against the dense fp16 cache of the same tokens.
            "physical_pool_bytes": physical,
            "physical_compression_x": dense / physical if physical else 0.0,
        }

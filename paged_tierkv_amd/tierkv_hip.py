"""Tiered paged decode attention on MI355X -- drop-in for tierkv_triton.

``tierkv_decode_attention`` keeps the signature, argument meaning, return
contract and exceptions of the reference wrapper (tierkv_triton.py:272-465):

* ValueError for a query that is not 4-D, batch != 1 with a 1-D table,
  query_len != 1, non-GPU tensors, dtypes other than fp16/bf16,
  ``num_blocks <= 0`` or ``num_blocks > block_table.shape[-1]``
  (tierkv_triton.py:291-304);
* RuntimeError when the HIP library is missing (tierkv_triton.py:267-269);
* returns ``(out [B, 1, H, D], None)`` or, with ``return_scores``,
  ``(out, score_sums)`` where ``score_sums`` is fp32 ``[H, max_blocks]``
  (``[B, H, max_blocks]`` for batched tables), zero past ``num_blocks``
  (tierkv_triton.py:371-377, .kiro bugfix contract).

Additive, keyword-only extensions:

* batched tables ``[B, max_blocks]`` with ``query [B, H, 1, D]`` and an
  optional per-sequence ``seq_num_blocks``;
* the WARM format is taken from the pools: uint8 codes + fp16 per-token
  scale/zero (the reference codec) or int8 codes + fp32 per-(slot, head)
  absmax scales (``k_zero``/``v_zero`` may be None);
* ``cold_mode``: ``"zero_logit"`` (reference: COLD tokens enter the softmax
  with K = V = 0) or ``"masked"`` (COLD blocks contribute nothing);
* ``splits``: split-K factor (default: chosen from the launch size).  The
  reference's ``TIERKV_SPLIT_DECODE`` switch is not needed: the kernel always
  splits when it pays, and the result equals the single pass up to fp32
  re-association;
* ``deterministic``: every wave takes a fixed share of its workgroup's tiles
  instead of taking tiles from a shared counter as it frees up, so the
  output is the same bits on every call over the same inputs (as the
  reference's Triton kernel is), for about 1-2 % of the launch time.  The
  default comes from ``TIERKV_DETERMINISTIC`` (off when unset);
* ``workspace``: a ``DecodeWorkspace`` the caller owns (a fixed one is
  required under HIP graph capture); by default each (device, stream) pair
  has its own implicit workspace, so launches on different streams never
  share scratch memory.  ``workspace=NOALLOC`` launches through
  ``tierkv_decode_attention_noalloc`` (the library's own 16 MiB device array
  per GPU, no allocation; launches on one GPU must not overlap).

``score_sums`` are reproducible: the same inputs give the same bits on every
launch (each block's statistics are staged on their own and reduced in a
fixed order), so tier labels ranked from them do not change from run to run.

Set ``TIERKV_CHECK_ERRORS=1`` to make every call synchronise and raise if
the kernel skipped a block whose slot or state was out of range.
"""

from __future__ import annotations

import ctypes
import os
import weakref

import torch

from . import _lib

NOALLOC = "noalloc"   # workspace= value: the allocation-free entry point


class DecodeWorkspace:
    """Device scratch of ``tierkv_decode_attention``: the error word, the
    split-arrival counters, the split partials and the per-block score stage.

    The kernels leave the counters at zero after every launch, so one
    workspace serves launches of any shape, and captured graphs can replay
    them -- as long as the launches that share it run one after another (on
    one stream, or otherwise ordered).

    ``growable=False`` fixes the buffer for the workspace's lifetime: a call
    that needs more raises instead of reallocating.  Captured graphs hold the
    buffer's address, so a workspace used under capture must be sized before
    the capture (``DecodeWorkspace.for_shape``); the first launch bound to a
    workspace under capture fixes it, so that no later eager launch can free
    memory a graph replays on.  A growable workspace replaces its buffer when
    a call needs more bytes; the error flags set in the old buffer are carried
    into the new one on the device (no host sync), and the old buffer is
    recorded on every stream that used it before it is dropped, so the
    caching allocator reuses it only after their queued work.  The reference
    caches one placeholder tensor per device the same way
    (tierkv_triton.py:24-40).
    """

    def __init__(self, device, nbytes: int = 0, *, growable: bool = True):
        self.device = torch.device(device)
        self.growable = bool(growable)
        self.buf = torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device=self.device)
        self._streams = []   # the streams launches bound to this workspace were issued on
        _LIVE.add(self)

    def note_stream(self, stream) -> None:
        """Record that launches on ``stream`` (a torch stream) use this workspace."""
        if self.device.type == "cuda" and all(stream != s for s in self._streams):
            self._streams.append(stream)

    @staticmethod
    def bytes_for(batch: int, num_heads: int, kv_heads: int, num_blocks: int, head_dim: int, *,
                  block_size: int = 16, return_scores: bool = True, splits: int = 0) -> int:
        need = _lib.lib().tierkv_decode_workspace_bytes(int(batch), int(num_heads), int(kv_heads), int(num_blocks),
                                                        int(block_size), int(head_dim), int(bool(return_scores)),
                                                        int(splits))
        if need < 0:
            raise ValueError("invalid decode geometry.")
        return int(need)

    @classmethod
    def for_shape(cls, device, batch: int, num_heads: int, kv_heads: int, num_blocks: int, head_dim: int, *,
                  block_size: int = 16, return_scores: bool = True, splits: int = 0) -> "DecodeWorkspace":
        """A fixed workspace large enough for every launch of this geometry
        with at most ``num_blocks`` blocks (with or without score sums)."""
        need = cls.bytes_for(batch, num_heads, kv_heads, num_blocks, head_dim, block_size=block_size,
                             return_scores=return_scores, splits=splits)
        return cls(device, need, growable=False)

    @property
    def nbytes(self) -> int:
        return int(self.buf.numel())

    def data_ptr(self) -> int:
        return self.buf.data_ptr()

    def _capturing(self) -> bool:
        return self.device.type == "cuda" and torch.cuda.is_current_stream_capturing()

    def reserve(self, nbytes: int) -> None:
        capturing = self._capturing()
        if nbytes <= self.nbytes:
            if capturing:
                self.growable = False   # a graph holds this buffer's address from now on
            return
        if capturing:
            raise RuntimeError("the decode workspace cannot grow during HIP graph capture: pass workspace= "
                               "(a DecodeWorkspace sized before the capture), or run the launch once eagerly "
                               "on this stream first.")
        if not self.growable:
            raise RuntimeError(f"decode workspace holds {self.nbytes} bytes, the launch needs {int(nbytes)}: "
                               "size the fixed workspace for the largest launch (DecodeWorkspace.for_shape).")
        new = torch.zeros(int(nbytes), dtype=torch.uint8, device=self.device)
        new[:4].view(torch.int32).bitwise_or_(self.buf[:4].view(torch.int32))
        if self.device.type == "cuda":
            current = torch.cuda.current_stream(self.device)
            for stream in self._streams + [current]:
                self.buf.record_stream(stream)
            self._streams = [current]
        self.buf = new

    def error_word(self, clear: bool = True) -> int:
        """The kernels' error flags (synchronises); cleared unless ``clear`` is False."""
        word = int(self.buf[:4].view(torch.int32).item())
        if word and clear:
            self.buf[:4].zero_()
        return word


_LIVE: "weakref.WeakSet[DecodeWorkspace]" = weakref.WeakSet()
# Implicit workspaces, one per (device, stream): launches on one stream are
# ordered, so they may share one; launches on different streams may overlap
# and never share.
_implicit: dict = {}


def stream_workspace(device=None) -> DecodeWorkspace:
    """The implicit workspace of torch's current stream on ``device``."""
    device = torch.device(device if device is not None else "cuda")
    if device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    key = (device.index, _lib.stream_of(device))
    ws = _implicit.get(key)
    if ws is None:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("no decode workspace exists for the capturing stream: pass workspace= (a "
                               "DecodeWorkspace sized before the capture).")
        ws = DecodeWorkspace(device)
        ws.note_stream(torch.cuda.current_stream(device))
        _implicit[key] = ws
    return ws


def noalloc_error_word(device, clear: bool = True) -> int:
    """The error flags of the allocation-free entry point's scratch on
    ``device`` (0 before its first launch there); synchronises the device."""
    device = torch.device(device)
    if device.type != "cuda":
        return 0
    word = ctypes.c_int32(0)
    with torch.cuda.device(device):
        _lib.check(_lib.lib().tierkv_decode_noalloc_error_word(int(bool(clear)), ctypes.addressof(word)),
                   "tierkv_decode_noalloc_error_word")
    return int(word.value)


def workspace_error_word(device) -> int:
    """Read (and clear) the kernels' error flags of every decode workspace on
    ``device`` and of the allocation-free scratch there (synchronises)."""
    device = torch.device(device)
    idx = device.index if device.index is not None else torch.cuda.current_device()
    word = 0
    for ws in list(_LIVE):
        if ws.device.type == device.type and (ws.device.index or 0) == idx:
            word |= ws.error_word()
    if device.type == "cuda":
        word |= noalloc_error_word(torch.device("cuda", idx))
    return word


def warm_format_of(warm_k_pool: torch.Tensor, k_scale: torch.Tensor) -> int:
    if warm_k_pool.dtype == torch.uint8 and k_scale.dtype == torch.float16:
        return _lib.WARM_REF_U8
    if warm_k_pool.dtype == torch.int8 and k_scale.dtype == torch.float32:
        return _lib.WARM_ABSMAX_I8
    raise ValueError(
        "WARM pools must be uint8 codes with fp16 scales (reference format) or int8 codes "
        "with fp32 per-(slot, head) scales (absmax format).")


_COLD_MODES = {"zero_logit": _lib.COLD_ZERO_LOGIT, "masked": _lib.COLD_MASKED}


def tierkv_decode_attention(
    query_states: torch.Tensor,
    block_table: torch.Tensor,
    block_states: torch.Tensor,
    block_lengths: torch.Tensor,
    hot_k_pool: torch.Tensor,
    hot_v_pool: torch.Tensor,
    warm_k_pool: torch.Tensor,
    warm_v_pool: torch.Tensor,
    k_scale: torch.Tensor,
    k_zero: torch.Tensor | None,
    v_scale: torch.Tensor,
    v_zero: torch.Tensor | None,
    num_blocks: int,
    num_key_value_groups: int,
    scaling: float,
    return_scores: bool = False,
    *,
    cold_mode: str = "zero_logit",
    seq_num_blocks=None,
    splits: int | None = None,
    workspace: DecodeWorkspace | None = None,
    deterministic: bool | None = None,
):
    """Decode attention over a tiered paged KV cache (see module docstring)."""
    lib = _lib.lib()  # RuntimeError if the HIP library is not built
    statics = (block_table, block_states, block_lengths, hot_k_pool, hot_v_pool, warm_k_pool, warm_v_pool,
               k_scale, k_zero, v_scale, v_zero)
    det = default_deterministic() if deterministic is None else bool(deterministic)
    simple = workspace is None and seq_num_blocks is None and splits is None
    if simple:
        hit = _rebind(lib, query_states, statics, num_blocks, num_key_value_groups, scaling, return_scores, cold_mode,
                      det)
        if hit is not None:
            args, out, score_sums, ws, batched = hit
            _launch(lib, args, query_states.device, ws)
            if score_sums is not None and not batched:
                score_sums = score_sums[0]
            return out, score_sums
    args, out, score_sums, ws, batched, _ = _bind(
        query_states, block_table, block_states, block_lengths, hot_k_pool, hot_v_pool, warm_k_pool, warm_v_pool,
        k_scale, k_zero, v_scale, v_zero, num_blocks, num_key_value_groups, scaling, return_scores,
        cold_mode=cold_mode, seq_num_blocks=seq_num_blocks, splits=splits, workspace=workspace, deterministic=det)
    if simple:
        _remember(query_states, statics, num_blocks, num_key_value_groups, scaling, return_scores, cold_mode, det,
                  args, batched)
    _launch(lib, args, query_states.device, ws)
    if score_sums is not None and not batched:
        score_sums = score_sums[0]
    return out, score_sums


# Calls that pass the same table, pool and metadata tensors again (a decode
# loop: the drop-in's per-layer launch every step) skip the validation of
# those tensors.  An entry holds them by weak reference and records their
# addresses; it matches only while every one is still the same live tensor at
# the same address, and everything that varies per call (the query, the block
# count, the output, the stream's workspace) is checked or made per call.
_REBIND: dict = {}
_REBIND_MAX = 64


def default_deterministic() -> bool:
    """The ``deterministic`` default: ``TIERKV_DETERMINISTIC`` set to a
    non-zero value."""
    return os.environ.get("TIERKV_DETERMINISTIC", "0") not in ("", "0")


def _rebind_key(query_states, statics, num_key_value_groups, scaling, return_scores, cold_mode, det):
    return (tuple(id(t) for t in statics), query_states.dtype, tuple(query_states.shape), query_states.device,
            int(num_key_value_groups), float(scaling), bool(return_scores), cold_mode, det)


def _remember(query_states, statics, num_blocks, num_key_value_groups, scaling, return_scores, cold_mode, det, args,
              batched):
    if len(_REBIND) >= _REBIND_MAX:
        _REBIND.pop(next(iter(_REBIND)))
    key = _rebind_key(query_states, statics, num_key_value_groups, scaling, return_scores, cold_mode, det)
    refs = tuple(None if t is None else weakref.ref(t) for t in statics)
    ptrs = tuple(None if t is None else t.data_ptr() for t in statics)
    # args: query, dtype, out, scores | table, states, lengths, stride, None | num_blocks | pools ... splits hint
    _REBIND[key] = (refs, ptrs, args[1], args[4:9], args[10:29], batched, {int(num_blocks): None})


def _rebind(lib, query_states, statics, num_blocks, num_key_value_groups, scaling, return_scores, cold_mode, det):
    """The bound arguments of a repeated call, or None (bind in full)."""
    if not _REBIND or not query_states.is_cuda:
        return None
    e = _REBIND.get(_rebind_key(query_states, statics, num_key_value_groups, scaling, return_scores, cold_mode,
                                det))
    if e is None:
        return None
    refs, ptrs, dtype_code, mid, tail, batched, needs = e
    for r, p, t in zip(refs, ptrs, statics):
        if (r is None) != (t is None) or (t is not None and (r() is not t or t.data_ptr() != p)):
            return None
    n = int(num_blocks)
    if n <= 0:
        raise ValueError("num_blocks must be positive.")
    if n > mid[3]:
        raise ValueError("num_blocks exceeds the provided block table length.")
    query = query_states.contiguous()
    batch, num_heads, _, head_dim = query.shape
    device = query.device
    out = torch.empty((batch, 1, num_heads, head_dim), device=device, dtype=query.dtype)
    score_sums = torch.empty((batch, num_heads, mid[3]), device=device, dtype=torch.float32) if return_scores else None
    need = needs.get(n)
    if need is None:
        # tail: hot_k, hot_v, hot_slots, warm_k, warm_v, warm_slots, k_scale, k_zero, v_scale, v_zero,
        # fmt, cold, batch, heads, kv_heads, block_size, head_dim, scaling, splits hint
        need = needs[n] = lib.tierkv_decode_workspace_bytes(batch, num_heads, tail[14], n, tail[15], head_dim,
                                                            int(return_scores), tail[18])
        if need < 0:
            raise ValueError("invalid decode geometry.")
    ws = stream_workspace(device)
    ws.reserve(need)
    args = ((_lib.ptr(query), dtype_code, _lib.ptr(out), _lib.ptr(score_sums)) + mid + (n,) + tail +
            (ws.data_ptr(), ws.nbytes))
    return args, out, score_sums, ws, batched


class PreparedDecode:
    """One ``tierkv_decode_attention`` launch validated and bound once, for
    loops that re-issue the same launch (a serving loop's layer step, a
    benchmark): ``launch()`` costs one C call on torch's current stream.

    The bound tensors must stay where they are; their contents may change
    between launches (write the next step's query into ``query`` in place).
    Every launch overwrites ``out`` (and ``score_sums``).  The launch owns a
    fixed workspace unless ``workspace`` (fixed) is given.  Arguments are
    those of ``tierkv_decode_attention``."""

    def __init__(self, *args, **kwargs):
        self._lib = _lib.lib()
        (self._args, self.out, scores, self.workspace, batched, self._keep) = _bind(*args, prepared=True, **kwargs)
        self.query = self._keep[0]   # the bound (contiguous) query tensor
        self.score_sums = scores if (scores is None or batched) else scores[0]
        self.device = self.out.device

    def launch(self):
        _launch(self._lib, self._args, self.device, self.workspace)
        return self.out, self.score_sums


def _bind(
    query_states: torch.Tensor,
    block_table: torch.Tensor,
    block_states: torch.Tensor,
    block_lengths: torch.Tensor,
    hot_k_pool: torch.Tensor,
    hot_v_pool: torch.Tensor,
    warm_k_pool: torch.Tensor,
    warm_v_pool: torch.Tensor,
    k_scale: torch.Tensor,
    k_zero: torch.Tensor | None,
    v_scale: torch.Tensor,
    v_zero: torch.Tensor | None,
    num_blocks: int,
    num_key_value_groups: int,
    scaling: float,
    return_scores: bool = False,
    *,
    cold_mode: str = "zero_logit",
    seq_num_blocks=None,
    splits: int | None = None,
    workspace: DecodeWorkspace | None = None,
    prepared: bool = False,
    deterministic: bool | None = None,
):
    """Validate one decode launch and bind its C-ABI arguments (all but the
    stream).  ``prepared`` binds a fixed workspace the launch owns unless one
    is given, so the bound pointers stay valid for every later launch."""
    lib = _lib.lib()  # RuntimeError if the HIP library is not built
    if query_states.ndim != 4:
        raise ValueError("query_states must have shape [batch, num_heads, query_len, head_dim].")
    batched = block_table.ndim == 2
    if not batched and query_states.shape[0] != 1:
        raise ValueError("TierKV decode supports batch size 1 only with a 1-D block table.")
    if query_states.shape[-2] != 1:
        raise ValueError("TierKV decode supports query_len == 1 only.")
    if not query_states.is_cuda:
        raise ValueError("TierKV decode requires GPU (HIP) tensors.")
    if query_states.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("TierKV decode supports fp16/bf16 query tensors only.")
    if int(num_blocks) <= 0:
        raise ValueError("num_blocks must be positive.")
    if int(num_blocks) > block_table.shape[-1]:
        raise ValueError("num_blocks exceeds the provided block table length.")
    if cold_mode not in _COLD_MODES:
        raise ValueError('cold_mode must be "zero_logit" or "masked".')

    batch, num_heads, _, head_dim = query_states.shape
    if batched and block_table.shape[0] != batch:
        raise ValueError("batched block tables must have one row per query batch entry.")
    for name, t in (("block_table", block_table), ("block_states", block_states),
                    ("block_lengths", block_lengths)):
        _lib.require_gpu_tensor(t, name)
        if t.dtype != torch.int32:
            raise ValueError(f"{name} must be int32.")
        # Batched tables share one row stride.  A 1-D table's states and
        # lengths are read at logical blocks [0, num_blocks) only, as the
        # reference kernel reads them (tierkv_triton.py:81-83): any length
        # covering them is accepted, e.g. a dense pool's per-block lengths.
        if batched or t.ndim != 1:
            if t.shape != block_table.shape:
                raise ValueError(f"{name} must have the block table's shape.")
        elif t.shape[0] < int(num_blocks):
            raise ValueError(f"{name} must have at least num_blocks entries.")
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous.")
    pools = (hot_k_pool, hot_v_pool, warm_k_pool, warm_v_pool)
    for name, t in zip(("hot_k_pool", "hot_v_pool", "warm_k_pool", "warm_v_pool"), pools):
        _lib.require_gpu_tensor(t, name)
        if t.ndim != 4 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous [slots, kv_heads, block_size, head_dim] tensor.")
    if hot_k_pool.dtype != torch.float16 or hot_v_pool.dtype != torch.float16:
        raise ValueError("HOT pools must be fp16.")
    kv_heads, block_size, pool_dim = (int(x) for x in hot_k_pool.shape[1:])
    if pool_dim != head_dim or tuple(warm_k_pool.shape[1:]) != (kv_heads, block_size, head_dim):
        raise ValueError("pool geometry does not match the query head_dim.")
    if hot_v_pool.shape != hot_k_pool.shape or warm_v_pool.shape != warm_k_pool.shape:
        raise ValueError("K and V pools must have identical shapes.")
    if kv_heads * int(num_key_value_groups) != num_heads:
        raise ValueError("num_heads must equal kv_heads * num_key_value_groups.")
    fmt = warm_format_of(warm_k_pool, k_scale)
    metas = (k_scale, v_scale) if fmt == _lib.WARM_ABSMAX_I8 else (k_scale, k_zero, v_scale, v_zero)
    for t in metas:
        if t is None:
            raise ValueError("reference-format WARM pools need k_zero and v_zero.")
        _lib.require_gpu_tensor(t, "warm metadata")
        if not t.is_contiguous() or t.shape[0] != warm_k_pool.shape[0]:
            raise ValueError("warm scale/zero tensors must be contiguous with one entry per WARM slot.")

    query = query_states.contiguous()
    table_stride = int(block_table.shape[-1])
    device = query.device
    out = torch.empty((batch, 1, num_heads, head_dim), device=device, dtype=query.dtype)
    score_sums = None
    if return_scores:
        score_sums = torch.empty((batch, num_heads, table_stride), device=device, dtype=torch.float32)

    snb = None
    if seq_num_blocks is not None:
        snb = torch.as_tensor(seq_num_blocks, dtype=torch.int32, device=device).contiguous()
        if snb.numel() != batch:
            raise ValueError("seq_num_blocks needs one entry per sequence.")

    splits_hint = int(splits) if splits else 0
    if not 0 <= splits_hint < _lib.DECODE_DETERMINISTIC:
        raise ValueError("splits must be a non-negative split factor.")
    if default_deterministic() if deterministic is None else deterministic:
        splits_hint |= _lib.DECODE_DETERMINISTIC
    need = lib.tierkv_decode_workspace_bytes(batch, num_heads, kv_heads, int(num_blocks), block_size,
                                             head_dim, int(return_scores), splits_hint)
    if need < 0:
        raise ValueError("invalid decode geometry.")
    if isinstance(workspace, str):
        if workspace != NOALLOC:
            raise ValueError(f"workspace must be a DecodeWorkspace, None or {NOALLOC!r}.")
        ws = None
    elif workspace is not None:
        ws = workspace
        ws.note_stream(torch.cuda.current_stream(device))
    elif prepared:
        ws = DecodeWorkspace(device, need, growable=False)
    else:
        ws = stream_workspace(device)
    if ws is not None:
        if ws.device != device:
            raise ValueError("the decode workspace lives on another device.")
        ws.reserve(need)
        if prepared and ws.growable:
            raise ValueError("a prepared decode needs a fixed workspace (DecodeWorkspace(..., growable=False)).")
    args = (
        _lib.ptr(query), _lib.DTYPE_BF16 if query.dtype == torch.bfloat16 else _lib.DTYPE_F16,
        _lib.ptr(out), _lib.ptr(score_sums),
        _lib.ptr(block_table), _lib.ptr(block_states), _lib.ptr(block_lengths), table_stride,
        _lib.ptr(snb), int(num_blocks),
        _lib.ptr(hot_k_pool), _lib.ptr(hot_v_pool), int(hot_k_pool.shape[0]),
        _lib.ptr(warm_k_pool), _lib.ptr(warm_v_pool), int(warm_k_pool.shape[0]),
        _lib.ptr(k_scale), _lib.ptr(k_zero) if fmt == _lib.WARM_REF_U8 else None,
        _lib.ptr(v_scale), _lib.ptr(v_zero) if fmt == _lib.WARM_REF_U8 else None,
        fmt, _COLD_MODES[cold_mode],
        batch, num_heads, kv_heads, block_size, head_dim,
        float(scaling), splits_hint)
    if ws is not None:
        args += (ws.data_ptr(), ws.nbytes)
    # The tensors whose addresses are bound stay referenced with the arguments.
    keep = (query, out, score_sums, snb, block_table, block_states, block_lengths, hot_k_pool, hot_v_pool,
            warm_k_pool, warm_v_pool, k_scale, k_zero, v_scale, v_zero, ws)
    return args, out, score_sums, ws, batched, keep


def _launch(lib, args, device, ws) -> None:
    if ws is None:
        rc = lib.tierkv_decode_attention_noalloc(*args, _lib.stream_of(device))
        _lib.check(rc, "tierkv_decode_attention_noalloc")
    else:
        rc = lib.tierkv_decode_attention(*args, _lib.stream_of(device))
        _lib.check(rc, "tierkv_decode_attention")
    if _lib.env_flag("TIERKV_CHECK_ERRORS"):
        word = noalloc_error_word(device) if ws is None else ws.error_word()
        if word:
            raise RuntimeError(f"TierKV decode skipped blocks with out-of-range slot/state (flag {word}).")



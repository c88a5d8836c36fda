"""BlockManager -- drop-in for the reference's native extension class.

Same constructor, methods, return types and RuntimeError behaviour as the
pybind11 ``BlockManager`` of csrc/block_manager.cpp:126-134; the logic lives
in the C++ of paged_tierkv_amd/csrc/block_manager.cpp behind the C ABI.
"""

from __future__ import annotations

import ctypes

from . import _lib


class BlockManager:
    def __init__(self, total_blocks: int = 100000):
        self._lib = _lib.lib()
        self._h = ctypes.c_void_p()
        rc = self._lib.tierkv_bm_create(int(total_blocks), ctypes.byref(self._h))
        self._check(rc)

    def _check(self, rc: int) -> None:
        if rc != _lib.TIERKV_OK:
            raise RuntimeError(_lib.last_error())

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._lib.tierkv_bm_destroy(h)
            self._h = None

    def allocate_block(self, seq_id: int) -> int:
        out = ctypes.c_int32()
        self._check(self._lib.tierkv_bm_allocate_block(self._h, int(seq_id), ctypes.byref(out)))
        return int(out.value)

    def free_sequence(self, seq_id: int) -> None:
        self._check(self._lib.tierkv_bm_free_sequence(self._h, int(seq_id)))

    def update_block_state(self, seq_id: int, logical_id: int, new_state: int) -> None:
        self._check(self._lib.tierkv_bm_update_block_state(self._h, int(seq_id), int(logical_id), int(new_state)))

    def set_block_states(self, seq_id: int, states) -> None:
        """Write the states of logical blocks [0, len(states)) at once."""
        arr = (ctypes.c_int32 * len(states))(*[int(s) for s in states])
        self._check(self._lib.tierkv_bm_set_block_states(self._h, int(seq_id), arr, len(states)))

    def num_blocks(self, seq_id: int) -> int:
        n = ctypes.c_int32()
        self._check(self._lib.tierkv_bm_num_blocks(self._h, int(seq_id), ctypes.byref(n)))
        return int(n.value)

    def _get(self, fn, seq_id: int) -> list[int]:
        n = self.num_blocks(seq_id)
        if n == 0:
            return []
        buf = (ctypes.c_int32 * n)()
        got = ctypes.c_int32()
        self._check(fn(self._h, int(seq_id), buf, n, ctypes.byref(got)))
        return list(buf[: got.value])

    def get_physical_indices(self, seq_id: int) -> list[int]:
        return self._get(self._lib.tierkv_bm_get_physical_indices, seq_id)

    def get_states(self, seq_id: int) -> list[int]:
        return self._get(self._lib.tierkv_bm_get_states, seq_id)

    def num_free(self) -> int:
        n = ctypes.c_int32()
        self._check(self._lib.tierkv_bm_num_free(self._h, ctypes.byref(n)))
        return int(n.value)

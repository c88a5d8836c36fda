"""Host-to-device transfer of small int32 arrays without a host sync.

Pool and runtime operations plan on the host (slot ids, table entries, copy
jobs) and hand the plan to a kernel.  A plain ``torch.tensor(..., device=)``
copies from pageable memory and synchronises the stream, which would put a
host sync on every decode step.  Instead each array is written into a slot of
a pinned ring buffer and copied asynchronously into the matching slot of a
device ring on the current stream:

* a pinned slot is rewritten only after the event recorded behind its last
  copy has completed (in steady state the wait finds it long done);
* a device slot is rewritten by a copy enqueued on the same stream after
  every kernel that read it, so stream order protects it.

All users of one device must stay on one stream, as the reference runtime
does (it launches everything on the current stream).
"""

from __future__ import annotations

import collections

import numpy as np
import torch

_SLOTS = 64
_SLOT_INTS = 16384          # 64 KB per slot; larger arrays take a one-off buffer


class _Ring:
    def __init__(self, device: torch.device):
        self.device = device
        self.host = torch.empty((_SLOTS, _SLOT_INTS), dtype=torch.int32, pin_memory=True)
        self.host_np = self.host.numpy()
        self.dev = torch.empty((_SLOTS, _SLOT_INTS), dtype=torch.int32, device=device)
        self.events = [torch.cuda.Event() for _ in range(_SLOTS)]
        self.recorded = [False] * _SLOTS
        self.next = 0
        self.big = collections.deque()     # (event, pinned buffer) of one-off copies in flight

    def _release_big(self) -> None:
        while self.big and self.big[0][0].query():
            self.big.popleft()

    def stage(self, arr: np.ndarray) -> torch.Tensor:
        arr = np.ascontiguousarray(arr, dtype=np.int32).reshape(-1)
        n = arr.size
        if n > _SLOT_INTS:
            self._release_big()
            pinned = torch.from_numpy(arr.copy()).pin_memory()
            out = torch.empty(n, dtype=torch.int32, device=self.device)
            out.copy_(pinned, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record()
            self.big.append((ev, pinned))
            return out
        i = self.next
        self.next = (i + 1) % _SLOTS
        ev = self.events[i]
        if self.recorded[i]:
            ev.synchronize()
        self.host_np[i, :n] = arr
        out = self.dev[i, :n]
        out.copy_(self.host[i, :n], non_blocking=True)
        ev.record()
        self.recorded[i] = True
        return out


_rings: dict = {}


def stage_i32(arr, device) -> torch.Tensor:
    """Copy an int32 host array to a device tensor valid for the kernels
    launched next on the current stream (see module docstring)."""
    device = torch.device(device)
    cur = torch.cuda.current_device()
    key = (device.type, device.index if device.index is not None else cur)
    ring = _rings.get(key)
    if ring is None:
        with torch.cuda.device(key[1]):
            ring = _Ring(torch.device("cuda", key[1]))
        _rings[key] = ring
    if key[1] == cur:
        return ring.stage(np.asarray(arr))
    with torch.cuda.device(key[1]):
        return ring.stage(np.asarray(arr))

"""BlockManager restatement (oracle; test infrastructure only).

Follows csrc/block_manager.cpp:22-124:

* the free list is filled total-1 .. 0 so ``pop`` hands out 0, 1, 2, ...
  (block_manager.cpp:30-33, 41-42);
* a new block is HOT with logical id = current sequence length (44-46);
* ``free_sequence`` pushes the sequence's physical ids back in logical order
  (LIFO reuse) and is a no-op for an unknown sequence (51-62);
* ``update_block_state`` raises on an unknown sequence, an out-of-range
  logical id or a state outside {0, 1, 2} (64-77, 108-119);
* getters return [] for an unknown sequence (79-105).

Pinned against the compiled reference (oracle/_ref, built from
csrc/block_manager.cpp by oracle/Makefile) on random operation sequences,
and by the reference's known answers (main.py:272-313).
"""

from __future__ import annotations


class BlockManagerOracle:
    def __init__(self, total_blocks: int = 100000):
        if total_blocks <= 0:
            raise RuntimeError("total_blocks must be positive")
        self.total_blocks = int(total_blocks)
        self.free_list = list(range(self.total_blocks - 1, -1, -1))
        self.table: dict[int, list[list[int]]] = {}   # seq -> [[physical, state], ...]

    def allocate_block(self, seq_id: int) -> int:
        if not self.free_list:
            raise RuntimeError("No free physical blocks available.")
        physical = self.free_list.pop()
        self.table.setdefault(int(seq_id), []).append([physical, 0])
        return physical

    def free_sequence(self, seq_id: int) -> None:
        blocks = self.table.pop(int(seq_id), None)
        if blocks is None:
            return
        for physical, _ in blocks:
            self.free_list.append(physical)

    def update_block_state(self, seq_id: int, logical_id: int, state: int) -> None:
        blocks = self.table.get(int(seq_id))
        if blocks is None:
            raise RuntimeError("Sequence not found for state update.")
        if logical_id < 0 or logical_id >= len(blocks):
            raise RuntimeError("Logical block ID out of range.")
        if state not in (0, 1, 2):
            raise RuntimeError("Invalid BlockState value.")
        blocks[logical_id][1] = int(state)

    def get_physical_indices(self, seq_id: int) -> list[int]:
        return [b[0] for b in self.table.get(int(seq_id), [])]

    def get_states(self, seq_id: int) -> list[int]:
        return [b[1] for b in self.table.get(int(seq_id), [])]

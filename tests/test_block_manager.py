"""Native BlockManager (C ABI) vs the reference: its known answers
(main.py:272-313), the compiled reference source in oracle/_ref
(csrc/block_manager.cpp built by oracle/Makefile) and the oracle
restatement, on random operation sequences (CPU)."""

from __future__ import annotations

import glob
import importlib.util
import os
import random

import pytest

from oracle.block_manager import BlockManagerOracle
from paged_tierkv_amd.block_manager import BlockManager

REF_DIR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref")


def _ref_module():
    hits = glob.glob(os.path.join(REF_DIR, "tierkv_ref_bm*.so"))
    if not hits:
        return None
    import torch  # noqa: F401  (the reference extension links libtorch)
    spec = importlib.util.spec_from_file_location("tierkv_ref_bm", hits[0])
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.mark.parametrize("cls", [BlockManager, BlockManagerOracle])
def test_reference_known_answers(cls):
    seq_id = 7
    manager = cls(total_blocks=8)
    assert [manager.allocate_block(seq_id) for _ in range(3)] == [0, 1, 2]
    assert manager.get_physical_indices(seq_id) == [0, 1, 2]
    manager.update_block_state(seq_id, 1, 1)
    assert manager.get_states(seq_id) == [0, 1, 0]
    overflow = cls(total_blocks=1)
    overflow.allocate_block(99)
    with pytest.raises(RuntimeError, match="No free physical blocks"):
        overflow.allocate_block(99)
    with pytest.raises(RuntimeError, match="Invalid BlockState"):
        manager.update_block_state(seq_id, 1, 9)
    with pytest.raises(RuntimeError, match="Logical block ID out of range"):
        manager.update_block_state(seq_id, 99, 1)
    with pytest.raises(RuntimeError, match="Sequence not found"):
        manager.update_block_state(12345, 0, 1)
    manager.free_sequence(-1)
    manager.free_sequence(seq_id)
    assert manager.get_physical_indices(seq_id) == []
    assert manager.get_states(seq_id) == []
    with pytest.raises(RuntimeError, match="total_blocks must be positive"):
        cls(total_blocks=0)


def _random_trace(managers, seed, steps=3000, total=64):
    rng = random.Random(seed)
    for _ in range(steps):
        op = rng.random()
        seq = rng.randrange(6)
        lid = rng.randrange(-1, 20)
        st = rng.randrange(-1, 4)
        results = []
        for m in managers:
            try:
                if op < 0.45:
                    results.append(("alloc", m.allocate_block(seq)))
                elif op < 0.55:
                    m.free_sequence(seq)
                    results.append(("free", None))
                elif op < 0.85:
                    m.update_block_state(seq, lid, st)
                    results.append(("upd", None))
                else:
                    results.append(("get", (m.get_physical_indices(seq), m.get_states(seq))))
            except RuntimeError as e:
                results.append(("err", str(e)))
        assert all(r == results[0] for r in results), results
    for seq in range(6):
        views = [(m.get_physical_indices(seq), m.get_states(seq)) for m in managers]
        assert all(v == views[0] for v in views)


def test_random_traces_match_oracle():
    for seed in range(5):
        _random_trace([BlockManager(total_blocks=64), BlockManagerOracle(total_blocks=64)], seed)


def test_random_traces_match_compiled_reference():
    ref = _ref_module()
    if ref is None:
        pytest.skip("oracle/_ref not built (needs the reference tree)")
    for seed in range(5):
        _random_trace([BlockManager(total_blocks=64), ref.BlockManager(total_blocks=64)], 100 + seed)


def test_batched_state_write():
    m = BlockManager(total_blocks=16)
    for _ in range(5):
        m.allocate_block(3)
    m.set_block_states(3, [0, 1, 2, 1])
    assert m.get_states(3) == [0, 1, 2, 1, 0]
    with pytest.raises(RuntimeError, match="Invalid BlockState"):
        m.set_block_states(3, [0, 7])
    assert m.get_states(3) == [0, 1, 2, 1, 0]      # all-or-nothing
    with pytest.raises(RuntimeError, match="out of range"):
        m.set_block_states(3, [0] * 6)
    assert m.num_free() == 11

"""Pins the CPU model of the batched runtime (oracle/runtime.py) against the
reference runtime's own recorded trajectories (tests/golden/runtime_*.npz,
written by the reference TieredKVRuntime, tierkv_policy.py:1534-1912).

One oracle instance per layer (the reference serves one sequence per
layer); prefill, appends and policy ticks are replayed with the recorded
inputs.  After every recorded operation the oracle's per-block tier states
and lengths must equal the reference's BlockManager states and length table
exactly.  Ticks take the recorded block scores directly (the block mass of
probability sums is pinned on its own by closed forms).

Slot ids of a batch are this build's own allocation order (the reference has
no batch); they are checked by invariants: every resident block owns a
distinct slot of its tier, and free stacks plus owned slots cover every slot
exactly once."""

from __future__ import annotations

import json
import os

import numpy as np
import pytest

from oracle.runtime import BatchedRuntimeOracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = ["runtime_compact_hot_warm", "runtime_compact_hot_warm_cold", "runtime_dense_hot_warm",
         "runtime_dense_hot_warm_cold"]
HOT_SLOTS = WARM_SLOTS = 64


def _invariants(orc: BatchedRuntimeOracle, where: str) -> None:
    n = int(orc.nb[0])
    for tier, free, cap in ((0, orc.hot_free, HOT_SLOTS), (1, orc.warm_free, WARM_SLOTS)):
        owned = [int(orc.table[0, i]) for i in range(n) if orc.states[0, i] == tier]
        assert len(set(owned)) == len(owned), f"{where}: tier {tier} slot shared"
        assert sorted(owned + list(free)) == list(range(cap)), f"{where}: tier {tier} slots lost or duplicated"
    cold = [i for i in range(n) if orc.states[0, i] == 2]
    assert all(orc.table[0, i] == -1 for i in cold), f"{where}: COLD block keeps a slot"


@pytest.mark.parametrize("name", CASES)
def test_oracle_runtime_follows_reference_trajectory(name):
    fx = np.load(os.path.join(GOLDEN, name + ".npz"))
    cfg = json.loads(str(fx["config"]))
    ops = json.loads(str(fx["ops"]))
    kv_all, scores_all = fx["kv"], fx["scores"]
    bs, hot_b, warm_b = cfg["block_size"], cfg["hot_budget"], cfg["warm_budget"]
    max_blocks = -(-cfg["max_seq_len"] // bs)
    mode = cfg["mode"]
    orcs = [BatchedRuntimeOracle(1, cfg["kv_heads"], cfg["head_dim"], bs, max_blocks, HOT_SLOTS, WARM_SLOTS,
                                 policy_mode=mode, warm_format="ref_u8") for _ in range(cfg["num_layers"])]
    len_row = 3 if cfg["layout"] == "compact" else 2
    checked = 0
    for op in ops:
        kind, where = op["op"], f"{name} op {op['i']} ({op['op']})"
        if kind == "prefill":
            off, t = op["kv"]
            k, v = kv_all[0, :, off:off + t][None], kv_all[1, :, off:off + t][None]
            so, sn = op["scores"]
            orcs[op["layer"]].prefill(k, v, scores_all[so:so + sn][None], hot_b, warm_b)
        elif kind == "append":
            off, t = op["kv"]
            for j in range(t):
                orcs[op["layer"]].append(kv_all[0, :, off + j:off + j + 1][None], kv_all[1, :, off + j:off + j + 1][None])
        elif kind == "policy":
            orc = orcs[op["layer"]]
            n = int(orc.nb[0])
            so, sn = op["scores"]
            assert sn == n, where
            orc.tick(None, hot_b, warm_b, scores=scores_all[so:so + sn].reshape(1, n))
        if "snap" in op and op.get("layer") is not None and kind in ("prefill", "append", "policy"):
            layer = op["layer"]
            orc = orcs[layer]
            n = int(orc.nb[0])
            want_states = op["snap"]["bm"][layer][1]
            assert orc.states[0, :n].tolist() == want_states, where
            want_len = op["snap"]["tables"][len_row][layer][:n]
            assert orc.lengths[0, :n].tolist() == want_len, where
            _invariants(orc, where)
            checked += 1
    assert checked > 60

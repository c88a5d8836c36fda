"""CPU oracle for the tiered paged KV-cache decode path.

TEST INFRASTRUCTURE ONLY.  Nothing in ``paged_tierkv_amd`` imports this
package: only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may use it, and only as the checker (or as the timed CPU
baseline), never as a product code path.

Every function restates the reference's algorithm (``/root/reference``,
xiaoMartintin/Paged_TierKV) in NumPy / plain Python and cites the file:line
it follows.  Modules:

* ``codec``         -- warm-tier quantizers: the reference's per-token
                       asymmetric uint8 codec and the per-(block, head)
                       symmetric int8 absmax codec.
* ``decode``        -- tiered paged decode attention (fp32 dequant, float64
                       softmax) with per-block probability sums.
* ``policy``        -- block scores, budget enforcement (tier labels), block
                       mass from probabilities.
* ``block_manager`` -- the native BlockManager's allocation/state rules.
* ``runtime``       -- the batched runtime's allocation order and tick rules
                       (per-sequence rules of the reference runtime; the
                       batch-level order is this build's own).

The reference-API pools and runtime (paged_tierkv_amd.tierkv_policy) have no
restatement here: they are pinned directly against trajectories the
reference runtime itself recorded (tests/golden/runtime_*.npz).

How each function is pinned (reference known answers, golden vectors written
by ``tests/golden/make_golden.py``, the compiled reference BlockManager in
``oracle/_ref``, closed forms, brute force, textbook identities) is listed in
the module docstrings; a function with no such check says "parity unpinned".
"""

HOT_STATE = 0
WARM_STATE = 1
COLD_STATE = 2

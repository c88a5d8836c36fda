"""The reference's own runtime-level tests, run against this build's drop-in
for its Python API (paged_tierkv_amd.tierkv_policy + BlockManager), with
the reference's inputs and assertions:

* test_tensor_pool_lazy_growth (main.py:408-449): the dense pool grows by
  whole chunks (2 -> 4 -> 6 blocks with chunk 2); WARM keeps the shape,
  COLD reconstructs to zeros, HOT round-trips exactly;
* test_tensor_pool_and_triton_decode (main.py:452-634): kernel decode
  against an eager reference over the reconstructed K/V (atol = rtol = 2e-2,
  the reference's tolerance), score sums [H, max_blocks] summing to 1 per
  head, a decode append without a full table sync, the decode-time
  reconstruction guard;
* test_policy_modes_and_scheduling (main.py:652-721): the first decode
  policy tick fires on step 64, ``every_step`` collects scores, and the
  three policy modes produce their tier sets;
* test_memory_telemetry_and_multi_runtime (main.py:724-776): per-runtime
  metrics and their aggregate."""

from __future__ import annotations

import pytest
import torch

from paged_tierkv_amd import tierkv_policy as tp
from paged_tierkv_amd.block_manager import BlockManager
from paged_tierkv_amd.tierkv_hip import tierkv_decode_attention

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _fresh_globals():
    tp.reset_global_tierkv()
    yield
    tp.reset_global_tierkv()


def test_tensor_pool_lazy_growth(device):
    print("[ref-scenario] pool lazy growth", flush=True)
    torch.manual_seed(0)
    pool = tp.TieredKVTensorPool(num_layers=1, block_size=4, max_seq_len=32, pool_chunk_blocks=2)
    k0, v0 = (torch.randn((1, 2, 4, 8), device=device, dtype=torch.float16) for _ in range(2))
    pool.store_hot_block(0, k0, v0)
    assert pool.allocated_pool_blocks == 2
    pool.demote_to_warm(0)
    k2, v2 = (torch.randn((1, 2, 4, 8), device=device, dtype=torch.float16) for _ in range(2))
    pool.store_hot_block(2, k2, v2)
    assert pool.allocated_pool_blocks == 4
    pool.demote_to_cold(2)
    k4, v4 = (torch.randn((1, 2, 4, 8), device=device, dtype=torch.float16) for _ in range(2))
    pool.store_hot_block(4, k4, v4)
    assert pool.allocated_pool_blocks == 6

    warm_k0, warm_v0 = pool.get_dequantized_block(0, tp.WARM_STATE)
    cold_k2, cold_v2 = pool.get_dequantized_block(2, tp.COLD_STATE)
    hot_k4, hot_v4 = pool.get_dequantized_block(4, tp.HOT_STATE)
    assert warm_k0.shape == k0.shape and warm_v0.shape == v0.shape
    assert torch.count_nonzero(cold_k2) == 0 and torch.count_nonzero(cold_v2) == 0
    assert torch.allclose(hot_k4, k4) and torch.allclose(hot_v4, v4)


def test_tensor_pool_and_kernel_decode(device):
    print("[ref-scenario] pool + kernel decode", flush=True)
    block_size, max_seq_len, kv_heads, q_heads, head_dim = 16, 64, 2, 4, 16
    groups = q_heads // kv_heads
    scaling = head_dim ** -0.5
    torch.manual_seed(1)

    def make_runtime(seq_len, seq_max_len=max_seq_len):
        tp.reset_global_tierkv()
        total = tp.estimate_pool_blocks(1, block_size, seq_max_len)
        cache = tp.initialize_global_tierkv(block_manager=BlockManager(total_blocks=total), num_layers=1,
                                            block_size=block_size, hot_budget=2, max_seq_len=seq_max_len,
                                            attention_backend="triton", pool_layout="dense")
        rt = cache.runtime
        k = torch.randn((1, kv_heads, seq_len, head_dim), device=device, dtype=torch.float16)
        v = torch.randn((1, kv_heads, seq_len, head_dim), device=device, dtype=torch.float16)
        rt.append_to_layer(0, k, v)
        return rt, k, v

    def reference_decode(q, k, v):
        # main.py:492-503: repeated K/V, softmax in fp32 rounded to the query dtype
        kk = k.repeat_interleave(groups, dim=1).float()
        vv = v.repeat_interleave(groups, dim=1).float()
        w = torch.softmax((q.float() @ kk.transpose(2, 3).contiguous()) * scaling, dim=-1).to(q.dtype)
        return (w.float() @ vv).transpose(1, 2).contiguous().to(q.dtype)

    def decode(rt, q, return_scores=False):
        table, states, lengths, n = rt.get_layer_table(0)
        pool = rt.kv_pool
        return tierkv_decode_attention(q, table, states, lengths, pool.hot_k_pool, pool.hot_v_pool,
                                       pool.warm_k_pool, pool.warm_v_pool, pool.k_scale, pool.k_zero,
                                       pool.v_scale, pool.v_zero, num_blocks=n, num_key_value_groups=groups,
                                       scaling=scaling, return_scores=return_scores)

    rt, k, v = make_runtime(21)
    rk, rv, phys, states = rt.reconstruct_layer(0)
    assert torch.allclose(rk, k) and torch.allclose(rv, v)
    assert [rt.kv_pool.get_block_length(i) for i in phys] == [16, 5]
    assert states == [tp.HOT_STATE, tp.HOT_STATE]
    q = torch.randn((1, q_heads, 1, head_dim), device=device, dtype=torch.float16)
    out, sums = decode(rt, q, return_scores=True)
    torch.testing.assert_close(out, reference_decode(q, k, v), atol=2e-2, rtol=2e-2)
    assert sums.shape == (q_heads, rt.max_blocks_per_layer)
    n = rt.layer_states[0].num_blocks
    torch.testing.assert_close(sums[:, :n].sum(-1), torch.ones(q_heads, device=device), atol=2e-2, rtol=0)
    syncs = rt.kv_pool.full_table_sync_count
    rt.append_to_layer(0, torch.randn((1, kv_heads, 1, head_dim), device=device, dtype=torch.float16),
                       torch.randn((1, kv_heads, 1, head_dim), device=device, dtype=torch.float16))
    assert rt.kv_pool.full_table_sync_count == syncs

    # All WARM (main.py:543-566).
    for logical in range(rt.layer_states[0].num_blocks):
        rt.block_manager.update_block_state(0, logical, tp.WARM_STATE)
    rt.sync_storage_states(0)
    wk, wv, _, _ = rt.reconstruct_layer(0)
    out_w, _ = decode(rt, q)
    torch.testing.assert_close(out_w, reference_decode(q, wk, wv), atol=2e-2, rtol=2e-2)

    # HOT / WARM / COLD (main.py:568-598): COLD reconstructs to zeros and
    # enters the softmax as zero logits, as in the reference kernel.
    rt, _, _ = make_runtime(41)
    rt.block_manager.update_block_state(0, 1, tp.WARM_STATE)
    rt.block_manager.update_block_state(0, 2, tp.COLD_STATE)
    rt.sync_storage_states(0)
    mk, mv, _, _ = rt.reconstruct_layer(0)
    out_m, _ = decode(rt, q)
    assert [rt.kv_pool.get_block_length(i) for i in rt.block_manager.get_physical_indices(0)] == [16, 16, 9]
    assert torch.count_nonzero(mk[:, :, -9:, :]) == 0 and torch.count_nonzero(mv[:, :, -9:, :]) == 0
    torch.testing.assert_close(out_m, reference_decode(q, mk, mv), atol=2e-2, rtol=2e-2)

    # More than four blocks (main.py:600-624).
    rt, _, _ = make_runtime(81, seq_max_len=128)
    for logical in (1, 3):
        rt.block_manager.update_block_state(0, logical, tp.WARM_STATE)
    rt.sync_storage_states(0)
    sk, sv, _, _ = rt.reconstruct_layer(0)
    assert rt.layer_states[0].num_blocks > 4
    out_s, _ = decode(rt, q)
    torch.testing.assert_close(out_s, reference_decode(q, sk, sv), atol=2e-2, rtol=2e-2)

    # Decode-time reconstruction is refused on the kernel path (main.py:626-631).
    rt.cache.begin_forward(1)
    with pytest.raises(RuntimeError):
        rt.reconstruct_layer(0)
    rt.cache.finish_forward()


def test_policy_modes_and_scheduling(device):
    print("[ref-scenario] policy modes and scheduling", flush=True)
    rt = tp.TieredKVRuntime(block_manager=BlockManager(total_blocks=128), num_layers=1, block_size=16, hot_budget=8,
                            max_seq_len=1024, policy_interval=64, policy_on_new_block=False,
                            score_accumulation_mode="policy_ticks", policy_mode="hot_warm")
    rt.begin_forward(1)
    assert not rt.should_run_decode_policy(0, allocated_new_block=True)
    assert not rt.should_collect_decode_scores(0, run_policy=False)
    rt.finish_forward()
    tick = False
    for _ in range(63):
        rt.begin_forward(1)
        tick = rt.should_run_decode_policy(0, allocated_new_block=False)
        rt.finish_forward()
    assert tick
    rt.score_accumulation_mode = "every_step"
    rt.begin_forward(1)
    assert rt.should_collect_decode_scores(0, run_policy=False)
    rt.finish_forward()

    def make_policy_runtime(mode, hot_budget=4, warm_budget=2, blocks=12):
        cache = tp.initialize_global_tierkv(block_manager=BlockManager(total_blocks=128), num_layers=1, block_size=16,
                                            hot_budget=hot_budget, max_seq_len=2048, policy_interval=16,
                                            policy_on_new_block=False, policy_mode=mode, warm_budget=warm_budget)
        r = cache.runtime
        for _ in range(blocks):
            r.block_manager.allocate_block(0)
        r.layer_states[0].num_blocks = blocks
        return r

    scores = torch.arange(12, device=device, dtype=torch.float32)
    hot = make_policy_runtime("hot_only")
    hot.enforce_policy(0, scores)
    assert set(hot.block_manager.get_states(0)) == {tp.HOT_STATE}
    warm = make_policy_runtime("hot_warm")
    warm.enforce_policy(0, scores)
    assert tp.WARM_STATE in set(warm.block_manager.get_states(0))
    tiered = make_policy_runtime("hot_warm_cold")
    tiered.enforce_policy(0, scores)
    states = set(tiered.block_manager.get_states(0))
    assert tp.WARM_STATE in states and tp.COLD_STATE in states


def test_memory_telemetry_and_multi_runtime(device):
    print("[ref-scenario] telemetry and multiple runtimes", flush=True)

    def make_runtime(seed):
        torch.manual_seed(seed)
        r = tp.create_tierkv_runtime(block_manager=BlockManager(total_blocks=16), num_layers=1, block_size=4,
                                     hot_budget=1, max_seq_len=32, attention_backend="triton", policy_interval=64,
                                     policy_on_new_block=False, policy_mode="hot_warm")
        k = torch.randn((1, 2, 9, 8), device=device, dtype=torch.float16)
        v = torch.randn((1, 2, 9, 8), device=device, dtype=torch.float16)
        r.append_to_layer(0, k, v)
        r.block_manager.update_block_state(0, 1, tp.WARM_STATE)
        r.sync_storage_states(0)
        return r

    a, b = make_runtime(11), make_runtime(13)
    ma, mb = a.collect_memory_metrics(), b.collect_memory_metrics()
    agg = tp.aggregate_memory_metrics([ma, mb])
    assert ma["hot_blocks"] > 0 and ma["warm_blocks"] > 0
    assert ma["logical_resident_mb"] > 0 and ma["logical_dense_equivalent_mb"] > 0
    assert 0 < ma["pool_utilization"] <= 1
    assert agg["hot_blocks"] == ma["hot_blocks"] + mb["hot_blocks"]
    assert agg["logical_resident_mb"] > ma["logical_resident_mb"]
    a.reset(release_storage=True)
    b.reset(release_storage=True)

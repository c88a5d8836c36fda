"""GPU parity of the tier-engine drop-in (paged_tierkv_amd.tierkv_policy)
against trajectories recorded from the reference runtime itself.

tests/golden/make_golden.py ran the reference TieredKVRuntime
(tierkv_policy.py:1534-1912) on the CPU over both pool layouts and both
tiering modes, with the reference BlockManager compiled from its own source,
and stored every input and the state after every operation.  Here the
drop-in replays the same operations on the GPU and must reproduce, exactly:

* the device tables (physical id / slot / state / length), free-slot lists,
  per-block dictionaries, BlockManager contents and layer states after every
  operation, and append_to_layer's return values;
* the SHA-256 of every pool tensor (HOT, WARM codes, scales, zero points,
  stale tails included) after prefill, after every policy tick and at the
  end, and the final pools byte for byte;
* reconstruct_layer's K/V and collect_memory_metrics.

block_scores_from_probability_sums is fp32 arithmetic whose reduction order
the reference leaves to ATen: compared within 1e-6 relative.  Finally the
decode kernel runs over the replayed tables through the reference's calling
convention (modeling_llama.py:433-456) and is compared with fp32 attention
over the reconstructed K/V, within the BASELINE tolerance."""

from __future__ import annotations

import importlib.util
import json
import os

import numpy as np
import pytest
import torch

from paged_tierkv_amd import tierkv_policy as tp
from paged_tierkv_amd.block_manager import BlockManager
from paged_tierkv_amd.tierkv_hip import tierkv_decode_attention

from helpers import ATOL, RTOL

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
# The last case has TinyLlama's attention geometry (4 kv heads, GQA group 8,
# head_dim 64, block 16): its decode launch runs the kernel's fast path
# (tiered_decode_kernel) over pools the reference wrote; the others (head_dim
# 16) run the generic path.
CASES = ["runtime_compact_hot_warm", "runtime_compact_hot_warm_cold", "runtime_dense_hot_warm",
         "runtime_dense_hot_warm_cold", "runtime_compact_hot_warm_cold_tinyllama"]


def _golden_module():
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(GOLDEN, "make_golden.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _replay(name, device):
    mg = _golden_module()
    fx = np.load(os.path.join(GOLDEN, name + ".npz"))
    cfg = json.loads(str(fx["config"]))
    ops = json.loads(str(fx["ops"]))
    kv_all = torch.from_numpy(fx["kv"]).to(device)
    scores_all = torch.from_numpy(fx["scores"])
    layout, mode = cfg["layout"], cfg["mode"]
    rt = tp.TieredKVRuntime(block_manager=BlockManager(total_blocks=256), num_layers=cfg["num_layers"],
                            block_size=cfg["block_size"], hot_budget=cfg["hot_budget"],
                            max_seq_len=cfg["max_seq_len"], attention_backend="eager",
                            policy_interval=cfg["policy_interval"], pool_chunk_blocks=cfg["pool_chunk_blocks"],
                            policy_on_new_block=False, score_accumulation_mode="policy_ticks", policy_mode=mode,
                            warm_budget=cfg["warm_budget"], pool_layout=layout)

    def kv(op):
        off, n = op["kv"]
        return kv_all[0, :, off:off + n][None], kv_all[1, :, off:off + n][None]

    def scores(op, dev):
        off, n = op["scores"]
        return scores_all[off:off + n].to(dev)

    for op in ops:
        kind, where = op["op"], f"{name} op {op['i']} ({op['op']})"
        if kind == "prefill":
            k, v = kv(op)
            # scores as a CPU tensor, as the reference's own tests pass them
            rt.append_prefill_with_policy(op["layer"], k, v, scores(op, "cpu"))
        elif kind == "begin":
            rt.cache.begin_forward(op["q"])
        elif kind == "finish":
            rt.cache.finish_forward()
        elif kind == "append":
            k, v = kv(op)
            got = rt.append_to_layer(op["layer"], k, v)
            assert got == op["ret"], where
            assert rt.should_run_decode_policy(op["layer"], got) == (ops[op["i"] + 1]["op"] == "policy"), where
        elif kind == "policy":
            rt.enforce_policy(op["layer"], scores(op, device))
            rt.sync_storage_states(op["layer"])
        elif kind == "resync":
            rt.sync_gpu_block_tables(op["layer"])
        elif kind == "score_sums":
            sums = torch.from_numpy(fx["score_sums"]).to(device)
            got = rt.block_scores_from_probability_sums(op["layer"], sums).cpu().numpy()
            np.testing.assert_allclose(got, fx["score_sums_out"], rtol=1e-6, atol=0, err_msg=where)
        elif kind == "reconstruct":
            key, val, _, _ = rt.reconstruct_layer(op["layer"])
            got = torch.stack([key[0], val[0]]).cpu().numpy()
            np.testing.assert_array_equal(got, fx[f"reconstruct_{op['layer']}"], err_msg=where)
        elif kind == "metrics":
            got = rt.collect_memory_metrics()
            assert set(got) == set(op["metrics"]), where
            for key, want in op["metrics"].items():
                assert got[key] == pytest.approx(want, rel=1e-12, abs=1e-12), f"{where}: {key}"
        else:
            raise AssertionError(f"unknown op {kind}")
        if "snap" in op:
            snap = mg.runtime_snapshot(rt, layout)
            for key, want in op["snap"].items():
                assert snap.get(key) == want, f"{where}: {key}\n got {snap.get(key)}\nwant {want}"
            assert set(snap) == set(op["snap"]), where
        if "digests" in op:
            for pname, want in op["digests"].items():
                assert mg.pool_digest(getattr(rt.kv_pool, pname)) == want, f"{where}: pool {pname}"
    for pname in mg.POOL_NAMES:
        t = getattr(rt.kv_pool, pname)
        if f"final_{pname}" in fx.files:
            np.testing.assert_array_equal(t.cpu().numpy(), fx[f"final_{pname}"], err_msg=f"{name}: final {pname}")
        else:
            assert t is None, pname
    return rt, cfg


@pytest.mark.parametrize("name", CASES)
def test_runtime_replays_reference_trajectory(device, name):
    print(f"[dropin] {name}", flush=True)
    rt, cfg = _replay(name, device)
    # Decode over the replayed tables, called the way the HF hook calls it.
    kvh, dim = cfg["kv_heads"], cfg["head_dim"]
    groups = cfg["heads"] // kvh
    gen = torch.Generator().manual_seed(5)
    for layer in range(cfg["num_layers"]):
        q = torch.randn((1, kvh * groups, 1, dim), generator=gen).half().to(device)
        table, states, lengths, n = rt.get_layer_table(layer)
        pool = rt.kv_pool
        out, sums = tierkv_decode_attention(q, table, states, lengths, pool.hot_k_pool, pool.hot_v_pool,
                                            pool.warm_k_pool, pool.warm_v_pool, pool.k_scale, pool.k_zero,
                                            pool.v_scale, pool.v_zero, num_blocks=n, num_key_value_groups=groups,
                                            scaling=dim ** -0.5, return_scores=True)
        key, val, _, _ = rt.reconstruct_layer(layer)
        kf = key[0].float().repeat_interleave(groups, dim=0)          # [H, T, D]
        vf = val[0].float().repeat_interleave(groups, dim=0)
        logits = (q[0].float() @ kf.transpose(1, 2)) * dim ** -0.5      # [H, 1, T]
        ref = (torch.softmax(logits, dim=-1) @ vf)[:, 0]                # [H, D]
        torch.testing.assert_close(out[0, 0].float(), ref, atol=ATOL, rtol=RTOL)
        assert sums.shape == (kvh * groups, table.shape[-1])
        torch.testing.assert_close(sums[:, :n].sum(dim=1), torch.ones(kvh * groups, device=device),
                                   atol=1e-3, rtol=0)
        bs = rt.block_scores_from_probability_sums(layer, sums)
        assert bs.shape == (n,)


def test_codec_functions_match_golden(device):
    """quantize_fp16_to_int8 / dequantize_int8_to_fp16 on the GPU against the
    reference's own outputs (arbitrary leading shape)."""
    fx = np.load(os.path.join(GOLDEN, "codec_ref_u8.npz"))
    x = torch.from_numpy(fx["x"]).to(device)
    q, s, z = tp.quantize_fp16_to_int8(x)
    np.testing.assert_array_equal(q.cpu().numpy(), fx["q"])
    np.testing.assert_array_equal(s.cpu().numpy(), fx["scale"])
    np.testing.assert_array_equal(z.cpu().numpy(), fx["zero"])
    d = tp.dequantize_int8_to_fp16(q, s, z)
    np.testing.assert_array_equal(d.cpu().numpy(), fx["deq"])
    # a shape whose row count is not a multiple of the 16-row tile
    q2, s2, z2 = tp.quantize_fp16_to_int8(x[:1, :3, :5])
    np.testing.assert_array_equal(q2.cpu().numpy(), fx["q"][:1, :3, :5])
    np.testing.assert_array_equal(s2.cpu().numpy(), fx["scale"][:1, :3, :5])


def test_pool_errors_match_reference(device):
    """Exception types and messages of the pool state machine
    (tierkv_policy.py:1042-1115, 934-967)."""
    pool = tp.CompactTieredKVTensorPool(num_layers=1, block_size=16, max_seq_len=64, max_hot_slots=2,
                                        max_warm_slots=1, hot_chunk_slots=1, warm_chunk_slots=1)
    k = torch.randn((1, 2, 16, 16), device=device).half()
    with pytest.raises(RuntimeError, match="has not been allocated"):
        pool.get_layer_table(0)
    pool.write_hot_tokens(0, 0, k, k)
    pool.promote_to_hot(0)                # HOT: no-op
    with pytest.raises(KeyError, match="not present in WARM storage"):
        pool.promote_to_hot(3)            # never stored
    pool.demote_to_warm(0)
    pool.demote_to_warm(0)                # WARM: no-op
    pool.demote_to_cold(0)
    with pytest.raises(KeyError, match="COLD"):
        pool.write_hot_tokens(0, 0, k, k)
    with pytest.raises(KeyError):
        pool.demote_to_cold(2)            # never stored
    with pytest.raises(ValueError, match="exceeds the physical block capacity"):
        pool.write_hot_tokens(1, 10, k[:, :, :8], k[:, :, :8])
    with pytest.raises(ValueError, match="cannot exceed block_size"):
        pool.write_hot_tokens(1, 0, torch.randn((1, 2, 17, 16), device=device).half(),
                              torch.randn((1, 2, 17, 16), device=device).half())
    with pytest.raises(RuntimeError, match="outside tensor-pool metadata capacity"):
        pool.write_hot_tokens(99, 0, k, k)
    pool.write_hot_tokens(1, 0, k, k)
    pool.write_hot_tokens(2, 0, k, k)
    with pytest.raises(RuntimeError, match="No HOT slots available"):
        pool.write_hot_tokens(3, 0, k, k)


@pytest.mark.parametrize("num_blocks", [4, 16, 64])
def test_reference_microbenchmark_call(device, num_blocks):
    """The call of the reference's own kernel microbenchmark
    (benchmark_no_score_anomaly, tierkv_triton.py:504-673): a dense
    TieredKVTensorPool with HOT blocks written by write_hot_tokens, a padded
    identity table, and the pool's per-block lengths (indexed by physical id,
    not of the table's length) passed as block_lengths.  Both return forms
    (tensor / None) and the output against fp32 attention over the written
    K/V."""
    bs, kvh, qh, d = 16, 4, 8, 64
    mb = num_blocks + 4
    gen = torch.Generator(device=device).manual_seed(num_blocks)
    pool = tp.TieredKVTensorPool(num_layers=1, block_size=bs, max_seq_len=mb * bs, max_blocks_per_layer=mb,
                                 pool_blocks=mb, pool_chunk_blocks=max(num_blocks, 4))
    ks, vs = [], []
    for phys in range(num_blocks):
        k = torch.randn((1, kvh, bs, d), generator=gen, device=device, dtype=torch.float16)
        v = torch.randn((1, kvh, bs, d), generator=gen, device=device, dtype=torch.float16)
        pool.write_hot_tokens(phys, 0, k, v)
        ks.append(k)
        vs.append(v)
    table = torch.full((mb,), -1, device=device, dtype=torch.int32)
    table[:num_blocks] = torch.arange(num_blocks, device=device, dtype=torch.int32)
    states = torch.full((mb,), tp.HOT_STATE, device=device, dtype=torch.int32)
    q = torch.randn((1, qh, 1, d), generator=gen, device=device, dtype=torch.float16)
    kw = dict(query_states=q, block_table=table, block_states=states, block_lengths=pool.block_lengths,
              hot_k_pool=pool.hot_k_pool, hot_v_pool=pool.hot_v_pool, warm_k_pool=pool.warm_k_pool,
              warm_v_pool=pool.warm_v_pool, k_scale=pool.k_scale, k_zero=pool.k_zero, v_scale=pool.v_scale,
              v_zero=pool.v_zero, num_blocks=num_blocks, num_key_value_groups=qh // kvh, scaling=d ** -0.5)
    print(f"[dropin] reference microbenchmark call, {num_blocks} blocks, lengths {tuple(pool.block_lengths.shape)}",
          flush=True)
    out_s, sums = tierkv_decode_attention(**kw, return_scores=True)
    out_n, none = tierkv_decode_attention(**kw, return_scores=False)
    torch.cuda.synchronize()
    assert none is None and sums is not None and sums.shape == (qh, mb)
    key = torch.cat(ks, dim=2)[0].float().repeat_interleave(qh // kvh, dim=0)      # [H, T, D]
    val = torch.cat(vs, dim=2)[0].float().repeat_interleave(qh // kvh, dim=0)
    p = torch.softmax((q[0].float() @ key.transpose(1, 2)) * d ** -0.5, dim=-1)   # [H, 1, T]
    ref = (p @ val)[:, 0]
    for out in (out_s, out_n):
        torch.testing.assert_close(out[0, 0].float(), ref, atol=ATOL, rtol=RTOL)
    blocks = p[:, 0].view(qh, num_blocks, bs).sum(-1)
    torch.testing.assert_close(sums[:, :num_blocks], blocks, atol=ATOL, rtol=RTOL)
    assert torch.count_nonzero(sums[:, num_blocks:]) == 0

"""Write golden vectors from the reference's own CPU code paths.

Run in the build container only (the reference tree is read, never copied):

    python tests/golden/make_golden.py /root/reference

Outputs small .npz fixtures next to this script:

* codec_ref_u8.npz -- quantize_fp16_to_int8 / dequantize_int8_to_fp16
  (tierkv_policy.py:21-44) on random fp16 rows plus edge rows (constant,
  all-positive, ties, wide range), executed by ATen on the CPU.  Pins the
  bit-exact fp16 op semantics the oracle codec restates.
* runtime_<layout>_<mode>.npz -- a scripted run of the reference runtime
  (TieredKVRuntime, tierkv_policy.py:1534-1912) over its pools
  (CompactTieredKVTensorPool 701-1365 / TieredKVTensorPool 53-698) with the
  reference BlockManager compiled from csrc/block_manager.cpp (oracle/_ref,
  built by oracle/Makefile): prefill with policy, single- and multi-token
  appends, policy ticks (enforce_policy + sync_storage_states), a table
  resync, score sums, reconstruction and memory metrics.  Stored: every
  input, the tables / free lists / per-block dictionaries after every
  operation, SHA-256 digests of every pool tensor at each checkpoint, and
  the final pools and outputs.  The ops list (JSON) is what the test
  replays against the drop-in.
* runtime_compact_hot_warm_cold_tinyllama.npz -- the same script at
  TinyLlama's attention geometry (4 kv heads, 32 q heads, head_dim 64,
  block 16), the shape the decode kernel's fast path serves, so the replay's
  decode launch over the reference-written pools runs that path.

``--only tinyllama`` writes just the last fixture.
"""

import glob
import hashlib
import importlib.util
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF_BM_DIR = os.path.join(os.path.dirname(os.path.dirname(HERE)), "oracle", "_ref")

# Runtime geometry of the trajectories (small enough for a fixture, every
# code path exercised).
TRAJ = dict(num_layers=2, kv_heads=2, head_dim=16, block_size=16, heads=4, hot_budget=4, warm_budget=3,
            max_seq_len=320, policy_interval=4, pool_chunk_blocks=16, prefill_tokens=90, steps=40)
# TinyLlama-1.1B's attention geometry, shorter run.
TRAJ_TINYLLAMA = dict(TRAJ, kv_heads=4, head_dim=64, heads=32, prefill_tokens=72, steps=24)
POOL_NAMES = ("hot_k_pool", "hot_v_pool", "warm_k_pool", "warm_v_pool", "k_scale", "k_zero", "v_scale", "v_zero")


def _ref_block_manager():
    hits = glob.glob(os.path.join(REF_BM_DIR, "tierkv_ref_bm*.so"))
    if not hits:
        raise SystemExit("build oracle/_ref first (make -C oracle)")
    spec = importlib.util.spec_from_file_location("tierkv_ref_bm", hits[0])
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.BlockManager


def pool_digest(t) -> str:
    if t is None:
        return ""
    a = np.ascontiguousarray(t.detach().cpu().numpy())
    return hashlib.sha256(str(a.dtype).encode() + str(a.shape).encode() + a.tobytes()).hexdigest()


def runtime_snapshot(rt, layout) -> dict:
    """Host-visible state of a runtime as JSON-ready int lists: tables, free
    lists, per-block dictionaries, BlockManager contents, layer states (the
    test reads the drop-in through the same function)."""
    pool = rt.kv_pool
    out = {}
    if pool.is_allocated():
        if layout == "compact":
            tabs = (pool.physical_block_tables, pool.block_slot_indices, pool.block_states, pool.block_lengths)
        else:
            tabs = (pool.block_tables, pool.block_states, pool.logical_block_lengths)
        out["tables"] = [t.detach().cpu().numpy().astype(np.int64).tolist() for t in tabs]
        if layout == "dense":
            out["phys_lengths"] = pool.block_lengths.detach().cpu().numpy().astype(np.int64).tolist()
    slots = getattr(pool, "physical_slots", {})
    lens = getattr(pool, "physical_lengths", {})
    out["phys"] = [[int(p), int(st), int(slots.get(p, -9)), int(lens.get(p, -9))]
                   for p, st in sorted(pool.physical_states.items())]
    if layout == "compact":
        out["hot_free"] = [int(x) for x in pool.hot_free_slots]
        out["warm_free"] = [int(x) for x in pool.warm_free_slots]
        out["alloc"] = [int(pool.allocated_hot_slots), int(pool.allocated_warm_slots)]
    else:
        out["alloc"] = [int(pool.allocated_pool_blocks)]
    bm = rt.block_manager
    out["bm"] = [[[int(x) for x in bm.get_physical_indices(l)], [int(x) for x in bm.get_states(l)]]
                 for l in range(rt.num_layers)]
    out["layers"] = [[int(ls.num_blocks), -1 if ls.open_physical_idx is None else int(ls.open_physical_idx),
                      int(ls.open_token_count)] for ls in (rt.layer_states[l] for l in range(rt.num_layers))]
    return out


def runtime_trajectory(tp, BM, layout, mode, seed, c=TRAJ):
    for key in list(os.environ):
        if key.startswith("TIERKV_"):
            del os.environ[key]
    g = torch.Generator().manual_seed(seed)
    rt = tp.TieredKVRuntime(block_manager=BM(total_blocks=256), num_layers=c["num_layers"],
                            block_size=c["block_size"], hot_budget=c["hot_budget"], max_seq_len=c["max_seq_len"],
                            attention_backend="eager", policy_interval=c["policy_interval"],
                            pool_chunk_blocks=c["pool_chunk_blocks"], policy_on_new_block=False,
                            score_accumulation_mode="policy_ticks", policy_mode=mode,
                            warm_budget=c["warm_budget"], pool_layout=layout)
    ops, arrays = [], {}
    kv_parts, score_parts = [], []          # inputs, concatenated along tokens / scores
    cursor = {"tok": 0, "score": 0}

    def add_kv(k, v):
        kv_parts.append(torch.stack([k[0], v[0]]).numpy())      # [2, kv, tokens, D]
        off = cursor["tok"]
        cursor["tok"] += int(k.shape[-2])
        return [off, int(k.shape[-2])]

    def add_scores(x):
        score_parts.append(x.numpy().astype(np.float32))
        off = cursor["score"]
        cursor["score"] += int(x.numel())
        return [off, int(x.numel())]

    def record(op, snap=True, digest=False):
        op["i"] = len(ops)
        if snap:
            op["snap"] = runtime_snapshot(rt, layout)
        if digest:
            op["digests"] = {n: pool_digest(getattr(rt.kv_pool, n)) for n in POOL_NAMES}
        ops.append(op)

    kv, dim, bs = c["kv_heads"], c["head_dim"], c["block_size"]
    T = c["prefill_tokens"]
    n0 = -(-T // bs)
    for layer in range(c["num_layers"]):
        k = torch.randn((1, kv, T, dim), generator=g).half()
        v = torch.randn((1, kv, T, dim), generator=g).half()
        scores = torch.rand(n0, generator=g)
        scores[2] = scores[3]                       # tie: the lower index ranks first
        rt.append_prefill_with_policy(layer, k, v, scores)
        record({"op": "prefill", "layer": layer, "kv": add_kv(k, v), "scores": add_scores(scores)}, digest=True)
    for step in range(c["steps"]):
        rt.cache.begin_forward(1)
        record({"op": "begin", "q": 1}, snap=False)
        for layer in range(c["num_layers"]):
            tokens = 20 if (step == 10 and layer == 1) else 1
            k = torch.randn((1, kv, tokens, dim), generator=g).half()
            v = torch.randn((1, kv, tokens, dim), generator=g).half()
            allocated = rt.append_to_layer(layer, k, v)
            record({"op": "append", "layer": layer, "ret": bool(allocated), "kv": add_kv(k, v)})
            if rt.should_run_decode_policy(layer, allocated):
                n = rt.layer_states[layer].num_blocks
                scores = torch.rand(n, generator=g)
                scores[n // 2] = scores[1]
                rt.enforce_policy(layer, scores)
                rt.sync_storage_states(layer)
                record({"op": "policy", "layer": layer, "scores": add_scores(scores)}, digest=True)
        rt.cache.finish_forward()
        record({"op": "finish"}, snap=False)
    for layer in range(c["num_layers"]):
        rt.sync_gpu_block_tables(layer)
        record({"op": "resync", "layer": layer})
    sums = torch.rand((c["heads"], rt.max_blocks_per_layer), generator=g)
    arrays["score_sums"] = sums.numpy()
    arrays["score_sums_out"] = rt.block_scores_from_probability_sums(0, sums).numpy()
    record({"op": "score_sums", "layer": 0}, snap=False)
    for layer in range(c["num_layers"]):
        key, val, _, _ = rt.reconstruct_layer(layer)
        arrays[f"reconstruct_{layer}"] = torch.stack([key[0], val[0]]).numpy()
        record({"op": "reconstruct", "layer": layer}, digest=True)
    metrics = rt.collect_memory_metrics()
    record({"op": "metrics", "metrics": {k: float(v) for k, v in metrics.items()}}, snap=False)
    for name in POOL_NAMES:
        t = getattr(rt.kv_pool, name)
        if t is not None:
            arrays[f"final_{name}"] = t.numpy()
    arrays["kv"] = np.concatenate(kv_parts, axis=2)
    arrays["scores"] = np.concatenate(score_parts)
    arrays["ops"] = np.array(json.dumps(ops))
    arrays["config"] = np.array(json.dumps(dict(c, layout=layout, mode=mode)))
    return arrays


def codec_vectors(tp):
    g = torch.Generator().manual_seed(1234)
    rows = [torch.randn((6, 4, 16, 64), generator=g).half()]
    edge = torch.zeros((1, 4, 16, 64), dtype=torch.float16)
    edge[0, 0] = 0.75                                      # constant rows -> scale 1
    edge[0, 1] = torch.linspace(1.0, 2.0, 64).half()       # all positive -> negative zp
    edge[0, 2] = (torch.arange(64) % 7).half() * 0.5       # many ties
    edge[0, 3] = torch.randn((16, 64), generator=g).half() * 40.0
    rows.append(edge)
    x = torch.cat(rows, dim=0)
    q, s, z = tp.quantize_fp16_to_int8(x)
    d = tp.dequantize_int8_to_fp16(q, s, z)
    return dict(x=x.numpy(), q=q.numpy(), scale=s.numpy(), zero=z.numpy(), deq=d.numpy())


def main(ref_root, only=None):
    sys.path.insert(0, ref_root)
    import tierkv_policy as tp   # the reference module, CPU only

    BM = _ref_block_manager()
    if only is None:
        np.savez_compressed(os.path.join(HERE, "codec_ref_u8.npz"), **codec_vectors(tp))
        print("wrote codec_ref_u8.npz")
        for seed, (layout, mode) in enumerate([("compact", "hot_warm"), ("compact", "hot_warm_cold"),
                                               ("dense", "hot_warm"), ("dense", "hot_warm_cold")]):
            name = f"runtime_{layout}_{mode}.npz"
            np.savez_compressed(os.path.join(HERE, name), **runtime_trajectory(tp, BM, layout, mode, 100 + seed))
            print("wrote", name)
    name = "runtime_compact_hot_warm_cold_tinyllama.npz"
    np.savez_compressed(os.path.join(HERE, name),
                        **runtime_trajectory(tp, BM, "compact", "hot_warm_cold", 200, TRAJ_TINYLLAMA))
    print("wrote", name)


if __name__ == "__main__":
    args = [a for a in sys.argv[1:] if not a.startswith("--")]
    only = sys.argv[sys.argv.index("--only") + 1] if "--only" in sys.argv else None
    if only is not None:
        args = [a for a in args if a != only]
    main(args[0] if args else "/root/reference", only)

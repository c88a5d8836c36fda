#!/usr/bin/env python3
"""Tiered paged decode-attention benchmark on one MI355X.

Workload (the metric's config): Llama-3-8B shape,
32 query / 8 KV heads, head_dim 128, batch 32, 4096-token contexts (256
blocks of 16), per sequence 26 HOT fp16 / 154 WARM int8-absmax / 76 COLD
(masked) blocks, slots shuffled across shared pools.  One step = one
decode-attention launch for one layer over the whole batch, with inputs
resident in HBM.  ``--layers`` distinct layer buffers (default 4, ~870 MB)
are rotated so the working set exceeds the 256 MB Infinity Cache.

Prints ONE JSON line.  ``value`` is algorithmic GB/s (ideal tiered bytes of
the step / step time); the line also carries us/layer-step, tokens/s
(attention-only, 32 layers), the HBM roofline fraction and a CPU baseline
(the oracle's NumPy restatement of the reference's eager decode, timed on a
bounded sample on this host).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
METRIC = "tiered decode-attn µs/layer + achieved HBM GB/s (% peak), Llama-3-8B shape"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=400)
    # Untimed launches before the timed region: the first ~500 launches after
    # idle run about 4% slower while the GPU's clocks settle.
    p.add_argument("--warmup", type=int, default=2000)
    p.add_argument("--layers", type=int, default=4)
    p.add_argument("--splits", type=int, default=0)
    p.add_argument("--workload", choices=["c3", "c4"], default="c3")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--mode", choices=["bench", "copy"], default="bench",
                   help="copy: time a plain device copy of known size (PMC calibration)")
    return p.parse_args()


def build_layers(args, device):
    import torch

    from paged_tierkv_amd import kernels, workloads as W

    layers = []
    gen = torch.Generator(device=device)
    for li in range(args.layers):
        mk = W.config3 if args.workload == "c3" else W.config4
        case = mk(seed=100 + li, with_data=False)
        gen.manual_seed(1000 + li)
        hs, ws = case.meta["hot_slots"], case.meta["warm_slots"]
        shp = (case.kv_heads, case.block_size, case.head_dim)
        hot_k = torch.randn((hs, *shp), generator=gen, device=device, dtype=torch.float16)
        hot_v = torch.randn((hs, *shp), generator=gen, device=device, dtype=torch.float16)
        warm_k = torch.empty((ws, *shp), device=device, dtype=torch.int8)
        warm_v = torch.empty((ws, *shp), device=device, dtype=torch.int8)
        k_scale = torch.empty((ws, case.kv_heads), device=device, dtype=torch.float32)
        v_scale = torch.empty((ws, case.kv_heads), device=device, dtype=torch.float32)
        src_k = torch.randn((ws, *shp), generator=gen, device=device, dtype=torch.float16)
        src_v = torch.randn((ws, *shp), generator=gen, device=device, dtype=torch.float16)
        idx = torch.arange(ws, dtype=torch.int32, device=device)
        kernels.demote_to_warm(src_k, src_v, idx, idx, torch.full((ws,), case.block_size, dtype=torch.int32),
                               warm_k, warm_v, k_scale, None, v_scale, None, warm_format="absmax_i8")
        torch.cuda.synchronize()
        del src_k, src_v
        layers.append(dict(
            case=case,
            args=dict(query_states=case.query.to(device), block_table=case.block_table.to(device),
                      block_states=case.block_states.to(device), block_lengths=case.block_lengths.to(device),
                      hot_k_pool=hot_k, hot_v_pool=hot_v, warm_k_pool=warm_k, warm_v_pool=warm_v,
                      k_scale=k_scale, k_zero=None, v_scale=v_scale, v_zero=None,
                      num_blocks=case.num_blocks, num_key_value_groups=case.groups, scaling=case.scaling)))
    return layers


def cpu_baseline(args, case_name):
    """Oracle decode (NumPy restatement of _eager_reference_decode) on one
    sequence of the same workload, repeated for ~cpu_seconds."""
    import numpy as np  # noqa: F401

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from helpers import oracle_decode, oracle_warm
    from paged_tierkv_amd import workloads as W

    mk = W.config3 if args.workload == "c3" else W.config4
    case = mk(seed=100, batch=1)
    warm = oracle_warm(case, "absmax_i8")
    nbytes = W.ideal_bytes(case.block_states, case.num_blocks, case.num_heads, case.kv_heads, case.head_dim)
    oracle_decode(case, warm, "absmax_i8", "masked")
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle_decode(case, warm, "absmax_i8", "masked")
        reps += 1
        el = time.perf_counter() - t0
        if el >= args.cpu_seconds:
            break
    per = el / reps
    return {"value": round(nbytes / per / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"1 of {32 if args.workload == 'c3' else 4} sequences of {case_name}, {reps} reps "
                      f"({per * 1e3:.1f} ms/sequence; NumPy, single thread)",
            "us_per_layer_step_extrapolated": round(per * 1e6 * (32 if args.workload == 'c3' else 4), 1)}


def copy_calibration(device):
    import torch

    n = 1 << 30
    a = torch.empty(n, dtype=torch.uint8, device=device)
    b = torch.empty(n, dtype=torch.uint8, device=device)
    a.fill_(1)
    for _ in range(20):
        b.copy_(a)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(20):
        b.copy_(a)
    e1.record()
    e1.synchronize()
    t = e0.elapsed_time(e1) / 1e3 / 20
    print(json.dumps({"mode": "copy", "bytes_read": n, "bytes_written": n, "sec": t,
                      "GBps_read_plus_write": 2 * n / t / 1e9}))


def main():
    args = parse()
    if args.gpus != 1:
        log("bench.py measures one GPU: every box in this pool has one MI355X, so --gpus must be 1.")
        sys.exit(2)
    import torch

    from paged_tierkv_amd import workloads as W
    from paged_tierkv_amd.tierkv_hip import tierkv_decode_attention, workspace_error_word

    device = torch.device("cuda:0")
    if args.mode == "copy":
        copy_calibration(device)
        return
    log(f"[bench] building {args.layers} layers of {args.workload} on {torch.cuda.get_device_name(0)}")
    layers = build_layers(args, device)
    case = layers[0]["case"]
    nbytes = W.ideal_bytes(case.block_states, case.num_blocks, case.num_heads, case.kv_heads, case.head_dim)
    splits = args.splits or None

    def step(i):
        tierkv_decode_attention(**layers[i % len(layers)]["args"], cold_mode="masked", splits=splits)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    assert workspace_error_word(device) == 0, "kernel flagged an out-of-range slot"
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(args.steps):
        step(i)
    e1.record()
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) / 1e3 / args.steps
    gbs = nbytes / sec / 1e9
    log(f"[bench] {sec * 1e6:.2f} us/layer-step, {gbs:.1f} GB/s algorithmic ({gbs / PEAK_HBM_GBS:.1%} of peak)")

    # HBM bytes per launch of the decode kernel from the committed rocprofv3
    # FETCH_SIZE / WRITE_SIZE summary of this workload (copy-calibrated).
    traffic = None
    tpath = os.path.join(ROOT, "profiles", f"tiered_decode_kernel_{case.name}_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] timing the CPU baseline")
        cpu = cpu_baseline(args, case.name)

    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": case.name, "batch": case.batch, "num_heads": case.num_heads,
                   "kv_heads": case.kv_heads, "head_dim": case.head_dim, "block_size": case.block_size,
                   "blocks_per_seq": case.num_blocks, "tiers_per_seq": list(case.tier_counts()[0]),
                   "warm_format": "int8 absmax per (block, kv head)", "cold": "masked",
                   "layers_rotated": args.layers},
        "us_per_layer_step": round(sec * 1e6, 3),
        "tokens_per_s_32_layers": round(case.batch / (32 * sec), 1),
        "ideal_bytes_per_step": nbytes,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

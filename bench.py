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
import statistics
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
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--layers", type=int, default=4)
    p.add_argument("--splits", type=int, default=0)
    p.add_argument("--workload", choices=["c3", "c1", "c4", "c2a", "promote", "c2b", "c5", "prefill", "ref",
                                          "microbench"],
                   default="c3",
                   help="c2a / promote / c2b: demotion / promotion / scoring microbenchmarks, c5: end-to-end random-init "
                        "Llama-3-8B decode through the HF hooks (each its own JSON line)")
    p.add_argument("--warm-format", choices=["absmax_i8", "ref_u8"], default="absmax_i8",
                   help="c3 / c4 / c2a / promote: WARM codec (BASELINE's int8 absmax, or the reference's uint8 "
                        "per-token)")
    p.add_argument("--cold", choices=["masked", "zero_logit"], default="masked",
                   help="c3 / c4: COLD semantics (BASELINE's masked eviction, or the reference's zero-logit tokens)")
    p.add_argument("--scores", action="store_true",
                   help="c3 / c4: the policy-step launch that also returns per-block probability sums")
    p.add_argument("--c5-steps", type=int, default=256)
    p.add_argument("--c5-batch", type=int, default=16)
    p.add_argument("--c5-prompt", type=int, default=2048)
    p.add_argument("--no-dense-baseline", action="store_true")
    p.add_argument("--ref-prompt", type=int, default=512, help="ref workload: prompt tokens (512/1024/1536/1900)")
    p.add_argument("--ref-steps", type=int, default=128, help="ref workload: greedy decode steps")
    p.add_argument("--c5-eager", action="store_true",
                   help="c5: run decode steps eagerly only (no HIP-graph replay, no eager comparison run)")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--deterministic", action="store_true",
                   help="decode workloads: fixed tile shares per wave (TIERKV_DECODE_DETERMINISTIC), so every "
                        "launch's output is the same bits")
    p.add_argument("--no-extras", action="store_true",
                   help="default C3 line: skip the extra decode figures (C3 with scores, C3 in the reference WARM "
                        "format, C4 with and without scores) timed after the headline")
    p.add_argument("--mode", choices=["bench", "copy", "ceiling"], default="bench",
                   help="copy: time a plain device copy of known size (PMC calibration); ceiling: HBM "
                        "stream-read and 4 KB-tile gather ceilings of the box")
    return p.parse_args()


def build_layers(args, device):
    """``--layers`` distinct layer buffers of the C3 / C4 workload, generated
    on the GPU from seeded generators; WARM tiles quantized on the GPU into
    the ``--warm-format`` pools (BASELINE's int8 absmax, or the reference's
    uint8 per-token codec)."""
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
        if args.warm_format == "absmax_i8":
            warm_k = torch.empty((ws, *shp), device=device, dtype=torch.int8)
            warm_v = torch.empty((ws, *shp), device=device, dtype=torch.int8)
            k_scale = torch.empty((ws, case.kv_heads), device=device, dtype=torch.float32)
            v_scale = torch.empty((ws, case.kv_heads), device=device, dtype=torch.float32)
            k_zero = v_zero = None
        else:
            warm_k = torch.empty((ws, *shp), device=device, dtype=torch.uint8)
            warm_v = torch.empty((ws, *shp), device=device, dtype=torch.uint8)
            meta = (ws, case.kv_heads, case.block_size, 1)
            k_scale, k_zero, v_scale, v_zero = (torch.empty(meta, device=device, dtype=torch.float16)
                                                for _ in range(4))
        src_k = torch.randn((ws, *shp), generator=gen, device=device, dtype=torch.float16)
        src_v = torch.randn((ws, *shp), generator=gen, device=device, dtype=torch.float16)
        idx = torch.arange(ws, dtype=torch.int32, device=device)
        kernels.demote_to_warm(src_k, src_v, idx, idx, torch.full((ws,), case.block_size, dtype=torch.int32),
                               warm_k, warm_v, k_scale, k_zero, v_scale, v_zero, warm_format=args.warm_format,
                               pad_tail=True)
        torch.cuda.synchronize()
        del src_k, src_v
        layers.append(dict(
            case=case,
            args=dict(query_states=case.query.to(device), block_table=case.block_table.to(device),
                      block_states=case.block_states.to(device), block_lengths=case.block_lengths.to(device),
                      hot_k_pool=hot_k, hot_v_pool=hot_v, warm_k_pool=warm_k, warm_v_pool=warm_v,
                      k_scale=k_scale, k_zero=k_zero, v_scale=v_scale, v_zero=v_zero,
                      num_blocks=case.num_blocks, num_key_value_groups=case.groups, scaling=case.scaling)))
    return layers


def cpu_host_info():
    """Threads for the CPU baseline and what the host reports: the box asks
    for at most 16 worker threads per GPU (OMP_NUM_THREADS), so the baseline
    uses min(os.cpu_count(), OMP_NUM_THREADS)."""
    import torch

    ncpu = os.cpu_count() or 1
    want = min(ncpu, int(os.environ.get("OMP_NUM_THREADS", ncpu) or ncpu))
    torch.set_num_threads(max(1, want))
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"os_cpu_count": ncpu, "torch_threads": torch.get_num_threads(), "cpu_model": model}


def cpu_baseline(args, layer, nbytes_fn):
    """The reference's CPU PyTorch decode path on this host
    (``oracle.torch_ref``): the restatement of _eager_reference_decode
    (tierkv_triton.py:708-820) with its per-block ``.item()`` loop,
    ``torch.cat``, ``repeat_interleave`` and fp32 softmax, looping over
    sequences as the reference serves a batch (main.py:1182-1189); and the
    vectorized torch-CPU variant beside it.  Inputs are layer 0's own tensors
    copied back from the GPU.  Each variant runs on a sample of the batch
    sized to about ``--cpu-seconds`` for 10 timed iterations after 2
    warm-ups, and both are checked against the NumPy oracle on that sample."""
    import numpy as np
    import torch

    from oracle import decode as odecode
    from oracle import torch_ref

    info = cpu_host_info()
    a = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in layer["args"].items()}
    case = layer["case"]
    cold = args.cold
    fmt = args.warm_format
    pos = (a["hot_k_pool"], a["hot_v_pool"], a["warm_k_pool"], a["warm_v_pool"], a["k_scale"], a["k_zero"],
           a["v_scale"], a["v_zero"], case.num_blocks, case.groups, case.scaling)

    def run(fn, seqs):
        return fn(a["query_states"][seqs], a["block_table"][seqs], a["block_states"][seqs], a["block_lengths"][seqs],
                  *pos, warm_format=fmt, cold_mode=cold)

    res = {}
    for name, fn in (("looped", torch_ref.eager_decode_looped), ("vectorized", torch_ref.vectorized_decode)):
        t0 = time.perf_counter()
        run(fn, slice(0, 1))
        t1 = time.perf_counter() - t0
        nseq = max(1, min(case.batch, int(args.cpu_seconds / 20 / max(t1, 1e-6))))
        seqs = slice(0, nseq)
        out = run(fn, seqs)
        reps, t0 = 0, time.perf_counter()
        while reps < 10:
            run(fn, seqs)
            reps += 1
        per = (time.perf_counter() - t0) / reps
        exp = odecode.decode_attention(
            a["query_states"][seqs, :, 0].numpy(), a["block_table"][seqs].numpy(), a["block_states"][seqs].numpy(),
            a["block_lengths"][seqs].numpy(), case.num_blocks,
            *(None if t is None else t.numpy() for t in pos[:8]), case.groups, case.scaling, warm_format=fmt,
            cold_mode=cold)
        err = np.abs(out[:, 0].float().numpy() - exp)
        if not (err <= 2e-3 + 1e-2 * np.abs(exp)).all():
            raise AssertionError(f"CPU baseline ({name}) disagrees with the oracle: max abs err {err.max():.3e}")
        nbytes = nbytes_fn(nseq)
        res[name] = {"GBps": round(nbytes / per / 1e9, 4), "sec_per_iter": round(per, 4), "seqs": nseq,
                     "us_per_layer_step_extrapolated": round(per / nseq * case.batch * 1e6, 1),
                     "max_abs_err_vs_oracle": float(err.max())}
        log(f"[bench] CPU {name}: {nseq} of {case.batch} sequences in {per * 1e3:.1f} ms "
            f"({res[name]['GBps']} GB/s algorithmic, {info['torch_threads']} threads)")
    lp = res["looped"]
    return {"value": lp["GBps"], "unit": "GB/s", "cores": info["torch_threads"], "kind": "port",
            "sample": (f"{lp['seqs']} of {case.batch} sequences of layer 0 of {case.name}, 10 iterations after 2 "
                       f"warm-ups: the reference's eager decode (tierkv_triton.py:708-820) restated in torch on "
                       f"the CPU (per-block .item() loop, torch.cat, repeat_interleave, fp32 softmax, a loop over "
                       f"sequences), checked against the NumPy oracle"),
            "us_per_layer_step_extrapolated": lp["us_per_layer_step_extrapolated"],
            "vectorized_torch_cpu": res["vectorized"], **info}


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


def ceiling(device, c3_bytes=216944640, stream_grids=(1024, 2048, 4096), reps=50, release=True):
    """HBM read ceilings of this box (libtierkv_ceiling.so): a non-temporal
    streaming read of 1 GiB, and a non-temporal gather of C3's ideal bytes
    (rounded to whole 4 KB tiles: 256 workgroups x 207 tiles) in a shuffled
    tile order out of the same 1 GiB buffer -- the decode kernel's access
    pattern without its arithmetic.  Each is timed with HIP events over
    ``reps`` launches after ``reps // 2`` untimed ones."""
    import ctypes

    import torch

    from paged_tierkv_amd import _lib, build as B

    lib = ctypes.CDLL(str(B.CEILING_LIB))
    for f in (lib.tierkv_ceiling_stream_read, lib.tierkv_ceiling_gather):
        f.restype = ctypes.c_int32
    lib.tierkv_ceiling_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int32,
                                               ctypes.c_void_p]
    lib.tierkv_ceiling_gather.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int32,
                                          ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p]
    n = 1 << 30
    src = torch.full((n,), 1, dtype=torch.uint8, device=device)
    sink = torch.zeros(4, dtype=torch.int32, device=device)
    stream = _lib.stream_of(device)
    n_wg = 256
    per_wg = c3_bytes // 4096 // n_wg
    gen = torch.Generator().manual_seed(7)
    order = torch.randperm(n // 4096, generator=gen)[:n_wg * per_wg].to(torch.int32).to(device)

    def timed(call, nbytes):
        for _ in range(max(reps // 2, 1)):
            assert call() == 0
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            call()
        e1.record()
        e1.synchronize()
        t = e0.elapsed_time(e1) / 1e3 / reps
        return t, nbytes / t / 1e9

    res = {"mode": "ceiling"}
    for grid in stream_grids:
        t, gbs = timed(lambda: lib.tierkv_ceiling_stream_read(src.data_ptr(), n, sink.data_ptr(), grid, stream), n)
        res[f"stream_read_grid{grid}_GBps"] = round(gbs, 1)
    gbytes = n_wg * per_wg * 4096
    t, gbs = timed(lambda: lib.tierkv_ceiling_gather(src.data_ptr(), n // 4096, order.data_ptr(), n_wg, per_wg,
                                                     sink.data_ptr(), stream), gbytes)
    res.update(gather_4k_tiles_bytes=gbytes, gather_4k_tiles_us=round(t * 1e6, 2), gather_4k_tiles_GBps=round(gbs, 1))
    del src, order
    if release:
        torch.cuda.empty_cache()
    return res


SETTLE_SEC = 0.06   # untimed decode launches before a decode line's warm-up steps


def settle(plans, seconds=SETTLE_SEC, at_least=0):
    """Keep the GPU launching ``plans`` (cycling) for at least ``seconds``
    and ``at_least`` launches; returns the number of launches.  The clocks
    follow the load with a lag: after the inputs are built (GPU idle) C3
    launches run 3-8 % slow for about 20 ms, and right after the ceiling
    measurement's streaming reads about 1 % slow for several milliseconds
    (measured on the box: 38.6 against 38.2 us for 20 timed steps).  A decode
    line's timed steps therefore follow this many untimed launches of the
    same kernel, so that they see the clocks of a decode loop.  The host
    synchronises every 200 launches, so the queue stays short."""
    import torch

    t0, i = time.perf_counter(), 0
    while i < at_least or time.perf_counter() - t0 < seconds:
        plans[i % len(plans)].launch()
        i += 1
        if i % 200 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return i


def graph_timed(fn, n_variants, steps, warmup, passes=1):
    """Average device time of fn(i) over `steps` calls (i cycling over
    n_variants input buffers): the launches of `passes` passes over the
    variants are captured once in a HIP graph, and replays are timed with HIP
    events on the current stream, so host launch cost stays outside the
    measurement."""
    import torch

    for i in range(max(warmup, n_variants)):
        fn(i % n_variants)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(passes):
            for i in range(n_variants):
                fn(i)
    n_variants *= passes
    reps = max(1, steps // n_variants)
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / (reps * n_variants), reps * n_variants


def _line(metric, value, unit, steps, warmup, sec, dtype, config, **extra):
    line = {"metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": steps, "warmup": warmup,
            "ms_per_step": round(sec * 1e3, 6), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": dtype, "data": "synthetic", "config": config}
    line.update(extra)
    return line


C1_METRIC = "tiered decode-attn µs per launch, TinyLlama shape, batch 1, 512-token context (latency-bound)"


def run_c1(args, device):
    """TinyLlama shape (32 q / 4 kv heads, head_dim
    64), batch 1, 512-token context: 8 HOT fp16 / 16 WARM int8-absmax / 8 COLD
    (masked) blocks in a dense pool of 64 blocks (physical ids shuffled).  It
    moves 271 KB, so a launch is latency-bound: the value is the time of one
    launch replayed from a HIP graph (host launch cost outside); the eager
    time (host launch included) is reported beside it."""
    import torch

    from paged_tierkv_amd import kernels, workloads as W
    from paged_tierkv_amd.tierkv_hip import PreparedDecode, tierkv_decode_attention, workspace_error_word

    case = W.config1()
    hot_k, hot_v = case.hot_k.to(device), case.hot_v.to(device)
    src_k, src_v = case.warm_src_k.to(device), case.warm_src_v.to(device)
    ns = src_k.shape[0]
    warm_k = torch.empty(src_k.shape, dtype=torch.int8, device=device)
    warm_v = torch.empty_like(warm_k)
    k_scale = torch.empty((ns, case.kv_heads), device=device)
    v_scale = torch.empty_like(k_scale)
    idx = torch.arange(ns, dtype=torch.int32, device=device)
    kernels.demote_to_warm(src_k, src_v, idx, idx, torch.full((ns,), case.block_size, dtype=torch.int32),
                           warm_k, warm_v, k_scale, None, v_scale, None, warm_format="absmax_i8")
    dargs = dict(query_states=case.query.to(device), block_table=case.block_table.to(device),
                 block_states=case.block_states.to(device), block_lengths=case.block_lengths.to(device),
                 hot_k_pool=hot_k, hot_v_pool=hot_v, warm_k_pool=warm_k, warm_v_pool=warm_v,
                 k_scale=k_scale, k_zero=None, v_scale=v_scale, v_zero=None,
                 num_blocks=case.num_blocks, num_key_value_groups=case.groups, scaling=case.scaling)

    def step(i):
        tierkv_decode_attention(**dargs, cold_mode="masked")

    # 50 launches per graph: a one-launch graph would time the graph launch.
    # The captured launch owns a fixed workspace (a capturing stream has no
    # implicit one).
    prepared = PreparedDecode(**dargs, cold_mode="masked")
    sec, steps = graph_timed(lambda i: prepared.launch(), 1, args.steps, 20, passes=50)
    for _ in range(20):
        step(0)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        step(0)
    e1.record()
    torch.cuda.synchronize()
    eager = e0.elapsed_time(e1) / 1e3 / args.steps
    assert workspace_error_word(device) == 0, "kernel flagged an out-of-range slot"
    nbytes = W.ideal_bytes(case.block_states, case.num_blocks, case.num_heads, case.kv_heads, case.head_dim)
    gbs = nbytes / sec / 1e9
    log(f"[c1] {sec * 1e6:.2f} us per launch (graph), {eager * 1e6:.2f} us eager; {gbs:.1f} GB/s algorithmic")
    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        from helpers import oracle_decode, oracle_warm

        warm = oracle_warm(case, "absmax_i8")
        oracle_decode(case, warm, "absmax_i8", "masked")
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds / 2:
            oracle_decode(case, warm, "absmax_i8", "masked")
            reps += 1
        per = (time.perf_counter() - t0) / reps
        cpu = {"value": round(per * 1e6, 1), "unit": "µs per launch", "cores": 1, "kind": "port",
               "sample": f"the whole C1 step, {reps} reps (oracle NumPy decode, single thread)"}
    cfg = {"workload": case.name, "batch": case.batch, "num_heads": case.num_heads, "kv_heads": case.kv_heads,
           "head_dim": case.head_dim, "block_size": case.block_size, "blocks_per_seq": case.num_blocks,
           "tiers_per_seq": list(case.tier_counts()[0]), "warm_format": "int8 absmax per (block, kv head)",
           "cold": "masked", "pool": "dense, 64 blocks"}
    line = _line(C1_METRIC, round(sec * 1e6, 3), "µs", steps, 20, sec, "f16", cfg,
                 us_eager=round(eager * 1e6, 3), ideal_bytes_per_step=nbytes,
                 roofline={"bound": "hbm", "achieved": round(gbs, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                           "frac": round(gbs / PEAK_HBM_GBS, 4),
                           "traffic": _profile_traffic("tiered_decode_kernel", case.name)},
                 cpu_baseline=cpu)
    line["higher_is_better"] = False
    print(json.dumps(line), flush=True)


PREFILL_METRIC = ("prefill block-score kernel TFLOP/s (% of the fp16 MFMA peak), C5 prefill shape: batch 16, "
                  "2048 tokens, 32 / 8 heads, head_dim 128")
PEAK_MFMA_F16_TFLOPS = 2500.0


def run_prefill(args, device):
    """The prefill block-score kernel (tierkv_prefill_block_mass: per-block
    causal attention mass of one layer's prefill, without materialised
    probabilities) at C5's prefill shape.  One step = one call for the whole
    batch.  Algorithmic FLOPs: two passes of q . k over the causal pairs,
    2 * 2 * B * H * T(T+1)/2 * D."""
    import torch

    from paged_tierkv_amd import kernels

    B, H, Hkv, T, D = args.c5_batch, 32, 8, args.c5_prompt, 128
    gen = torch.Generator(device=device).manual_seed(4000)
    qs = [torch.randn((B, H, T, D), generator=gen, device=device, dtype=torch.float16) for _ in range(2)]
    ks = [torch.randn((B, Hkv, T, D), generator=gen, device=device, dtype=torch.float16) for _ in range(2)]
    scaling = D ** -0.5

    def step(i):
        kernels.prefill_block_mass(qs[i % 2], ks[i % 2], 16, scaling)

    # at least 3 calls and 100 ms of them, so the clocks have settled
    t0, i = time.perf_counter(), 0
    while i < 3 or time.perf_counter() - t0 < 0.1:
        step(i)
        i += 1
        if i % 20 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    steps = max(4, min(args.steps, 20))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        step(i)
    e1.record()
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) / 1e3 / steps
    flops = 2 * 2 * B * H * (T * (T + 1) // 2) * D
    tf = flops / sec / 1e12
    log(f"[prefill] {sec * 1e3:.3f} ms per call, {tf:.1f} TFLOP/s ({tf / PEAK_MFMA_F16_TFLOPS:.1%} of the fp16 peak)")
    cpu = None
    if not args.no_cpu_baseline:
        import numpy as np
        from threadpoolctl import threadpool_limits

        from oracle.policy import prefill_block_mass as oracle_mass

        G = H // Hkv
        qn = qs[0][:1, :G].float().cpu().numpy()
        kn = ks[0][:1, :1].float().cpu().numpy()
        with threadpool_limits(1):
            t0 = time.perf_counter()
            oracle_mass(qn, kn, scaling, 16)
            per = time.perf_counter() - t0
        sflops = 2 * 2 * G * (T * (T + 1) // 2) * D
        cpu = {"value": round(sflops / per / 1e12, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
               "sample": f"one sequence, one kv head ({G} q heads) of the batch, {per:.1f} s "
                         "(oracle NumPy float64 probabilities, single thread)"}
    cfg = {"workload": "prefill_block_mass_c5", "batch": B, "num_heads": H, "kv_heads": Hkv, "tokens": T,
           "head_dim": D, "block_size": 16}
    print(json.dumps(_line(PREFILL_METRIC, round(tf, 2), "TFLOP/s", steps, 3, sec, "f16", cfg,
                           ms_per_call=round(sec * 1e3, 4), algorithmic_flops=flops,
                           roofline={"kernel": "prefill_block_mass_kernel", "bound": "mfma", "achieved": round(tf, 2),
                                     "peak": PEAK_MFMA_F16_TFLOPS, "unit": "TFLOP/s",
                                     "frac": round(tf / PEAK_MFMA_F16_TFLOPS, 4), "traffic": None},
                           cpu_baseline=cpu)), flush=True)


C2A_METRIC = "demotion HOT fp16 -> WARM int8 absmax GB/s (% peak), Llama-3-8B KV shape, 2048 of 4096 blocks"
CODEC_METRICS = {
    ("demote", "ref_u8"): "demotion HOT fp16 -> WARM uint8 (reference per-token codec) GB/s (% peak), Llama-3-8B "
                          "KV shape, 2048 of 4096 blocks",
    ("promote", "absmax_i8"): "promotion WARM int8 absmax -> HOT fp16 GB/s (% peak), Llama-3-8B KV shape, 2048 blocks",
    ("promote", "ref_u8"): "promotion WARM uint8 (reference per-token codec) -> HOT fp16 GB/s (% peak), Llama-3-8B "
                           "KV shape, 2048 blocks",
}
C2B_METRIC = "block-score + tier-label µs per call, probs [32, 32, 4096] -> per-block mass [32, 256] + labels"


def run_c2a(args, device):
    """BASELINE.json configs[1](a): quantize a seeded 50 % of a 4096-block
    fp16 pool (8 kv heads, 16 x 128) into WARM slots, table/state rewrite
    fused.  One step = one launch; 3 source pools are rotated (805 MB).

    ``--warm-format`` picks the codec: int8 absmax with fp32 per-(block,
    head) scales (BASELINE's), or the reference's uint8 with fp16 per-token
    scale and zero point (quantize_fp16_to_int8, tierkv_policy.py:21-36).
    ``--workload promote`` times the way back (promote_to_hot,
    tierkv_policy.py:1087-1115): the same 2048 blocks dequantized from 3
    rotated WARM sets into HOT slots, table/state rewrite fused."""
    import torch

    from paged_tierkv_amd import kernels, workloads as W

    fmt = args.warm_format
    op = "promote" if args.workload == "promote" else "demote"
    case = W.config2a()
    n = len(case.demote_logical)
    H, bs, D = 8, 16, 128
    pools = []
    gen = torch.Generator(device=device)
    for li in range(3):
        gen.manual_seed(2000 + li)
        shp = (case.hot_k.shape[0], H, bs, D)
        pools.append((torch.randn(shp, generator=gen, device=device, dtype=torch.float16),
                      torch.randn(shp, generator=gen, device=device, dtype=torch.float16)))
    del case.hot_k, case.hot_v
    src = case.table[0, case.demote_logical].to(device)
    dst = case.warm_slots.to(device)
    lens = torch.full((n,), bs, dtype=torch.int32, device=device)
    pos = case.demote_logical.to(torch.int32).to(device)
    table, states = case.table.to(device), case.states.to(device)

    def warm_set():
        wk = torch.empty((n, H, bs, D), dtype=torch.int8 if fmt == "absmax_i8" else torch.uint8, device=device)
        if fmt == "absmax_i8":
            meta = (torch.empty((n, H), device=device), None, torch.empty((n, H), device=device), None)
        else:
            meta = tuple(torch.empty((n, H, bs, 1), dtype=torch.float16, device=device) for _ in range(4))
        return wk, torch.empty_like(wk), meta

    def demote(i, w):
        kernels.demote_to_warm(pools[i][0], pools[i][1], src, dst, lens, w[0], w[1], *w[2], warm_format=fmt,
                               block_table=table, block_states=states, table_pos=pos)

    if op == "demote":
        w0 = warm_set()
        step = lambda i: demote(i % len(pools), w0)
        kernel = "demote_absmax_wave_kernel" if fmt == "absmax_i8" else "demote_ref_wave_kernel"
        nbytes = W.codec_ideal_bytes(n, H, bs, D, fmt, "demote")
    else:
        sets = [warm_set() for _ in range(3)]
        for i, w in enumerate(sets):
            demote(i, w)
        hot_dst = torch.arange(n, dtype=torch.int32, device=device)
        out_k = pools[0][0]                      # promoted into the first n slots of a HOT pool

        def step(i):
            w = sets[i % len(sets)]
            kernels.promote_to_hot(w[0], w[1], *w[2], dst, hot_dst, lens, out_k, pools[0][1], warm_format=fmt,
                                   block_table=table, block_states=states, table_pos=pos)
        kernel = "promote_wave_kernel"
        nbytes = W.codec_ideal_bytes(n, H, bs, D, fmt, "promote")

    # Eager launches: the host enqueues faster than one launch runs (~38 us),
    # so back-to-back launches time the kernel itself.
    for i in range(200):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(args.steps):
        step(i)
    e1.record()
    torch.cuda.synchronize()
    sec, steps = e0.elapsed_time(e1) / 1e3 / args.steps, args.steps
    gbs = nbytes / sec / 1e9
    log(f"[{op} {fmt}] {sec * 1e6:.2f} us per launch, {gbs:.1f} GB/s ({gbs / PEAK_HBM_GBS:.1%} of peak)")
    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, ROOT)
        from oracle import codec

        sample = pools[0][0][src[:128].long()].cpu().numpy()
        if op == "demote":
            fn = (lambda: codec.quantize_absmax_i8(sample)) if fmt == "absmax_i8" else \
                (lambda: codec.quantize_ref_u8(sample))
        else:
            if fmt == "absmax_i8":
                qs = codec.quantize_absmax_i8(sample)
                fn = lambda: codec.dequantize_absmax_i8(*qs).astype("float16")
            else:
                qs = codec.quantize_ref_u8(sample)
                fn = lambda: codec.dequantize_ref_u8(*qs)
        fn()
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds / 2:
            fn()
            reps += 1
        per_tile_set = (time.perf_counter() - t0) / reps
        cpu_gbs = W.codec_ideal_bytes(128, H, bs, D, fmt, op) / 2 / per_tile_set / 1e9
        cpu = {"value": round(cpu_gbs, 4), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"K tiles of 128 of the {n} blocks, {reps} reps ({per_tile_set * 1e3:.1f} ms; oracle "
                         f"NumPy {fmt} codec, {'quantize' if op == 'demote' else 'dequantize'}, single thread)"}
    fmt_name = "int8 absmax per (block, kv head)" if fmt == "absmax_i8" else \
        "reference uint8, fp16 scale and zero point per (token, kv head)"
    if op == "demote" and fmt == "absmax_i8":
        workload, metric = "c2a_demote_llama3_8b_kv", C2A_METRIC
    else:
        workload, metric = f"c2a_{op}_{fmt}_llama3_8b_kv", CODEC_METRICS[(op, fmt)]
    cfg = {"workload": workload, "pool_blocks": int(table.shape[1]), f"{op}d_blocks": n,
           "kv_heads": H, "block_size": bs, "head_dim": D, "warm_format": fmt_name,
           ("source_pools_rotated" if op == "demote" else "warm_sets_rotated"): 3}
    dtype = ("f16->i8" if fmt == "absmax_i8" else "f16->u8") if op == "demote" else \
        ("i8->f16" if fmt == "absmax_i8" else "u8->f16")
    print(json.dumps(_line(metric, round(gbs, 2), "GB/s", steps, 200, sec, dtype, cfg,
                           us_per_call=round(sec * 1e6, 3), ideal_bytes_per_step=nbytes,
                           roofline={"kernel": kernel, "bound": "hbm",
                                     "achieved": round(gbs, 2), "peak": PEAK_HBM_GBS,
                                     "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                                     "traffic": _profile_traffic(kernel, workload)},
                           cpu_baseline=cpu)), flush=True)


def run_c2b(args, device):
    """BASELINE.json configs[1](b): per-block probability mass of fp32
    probabilities [32, 32, 4096] and top-k HOT / bottom-k COLD tier labels
    (26 HOT incl. blocks 0 and 255, 77 COLD).  One step = the block-mass
    launch plus the label launch; 20 probability buffers are rotated
    (336 MB)."""
    import numpy as np
    import torch

    from paged_tierkv_amd import kernels, workloads as W

    base = W.config2b().to(device)
    bufs = [base] + [torch.softmax(torch.randn(base.shape, generator=torch.Generator(device=device).manual_seed(3000 + i),
                                               device=device) * 3.0, dim=-1) for i in range(19)]
    B, H, T = base.shape
    nblk = T // 16
    mass = torch.empty((B, nblk), device=device)
    cur = torch.zeros((B, nblk), dtype=torch.int32, device=device)
    labels = torch.empty_like(cur)

    def step(i):
        kernels.block_mass_from_probs(bufs[i], 16, out=mass)
        kernels.tier_labels(mass, cur, W.C2B_HOT_BUDGET, W.C2B_WARM_BUDGET, "hot_warm_cold", out=labels)

    sec, steps = graph_timed(step, len(bufs), args.steps, 20)
    # The dominant kernel (block mass: all but 0.1 % of the bytes) alone.
    msec, _ = graph_timed(lambda i: kernels.block_mass_from_probs(bufs[i], 16, out=mass), len(bufs), args.steps, 20)
    nbytes = W.score_ideal_bytes(B, H, T, 16)
    mbytes = B * H * T * 4 + B * nblk * 4
    gbs = mbytes / msec / 1e9
    log(f"[c2b] {sec * 1e6:.2f} us per scoring step (mass + labels); mass kernel {msec * 1e6:.2f} us, "
        f"{gbs:.1f} GB/s ({gbs / PEAK_HBM_GBS:.1%} of peak)")
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import policy as opolicy

        p = base.cpu().numpy()
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds / 2:
            m = opolicy.block_mass_from_probs(p, 16)
            opolicy.tier_labels(m, np.zeros((B, nblk), np.int32), W.C2B_HOT_BUDGET, W.C2B_WARM_BUDGET,
                                "hot_warm_cold")
            reps += 1
        per = (time.perf_counter() - t0) / reps
        cpu = {"value": round(per * 1e6, 1), "unit": "µs per call", "cores": 1, "kind": "port",
               "sample": f"the full C2(b) input, {reps} reps (oracle NumPy block mass + stable-rank labels, "
                         f"single thread)"}
    cfg = {"workload": "c2b_block_score_labels", "batch": B, "num_heads": H, "tokens": T, "block_size": 16,
           "hot_budget": W.C2B_HOT_BUDGET, "warm_budget": W.C2B_WARM_BUDGET, "prob_buffers_rotated": len(bufs)}
    line = _line(C2B_METRIC, round(sec * 1e6, 3), "µs", steps, 20, sec, "f32", cfg,
                 ideal_bytes_per_step=nbytes, block_mass_us=round(msec * 1e6, 3),
                 roofline={"kernel": "block_mass_staged_kernel", "bound": "hbm", "achieved": round(gbs, 2),
                           "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                           "traffic": _profile_traffic("block_mass_staged_kernel", cfg["workload"])},
                 cpu_baseline=cpu)
    line["higher_is_better"] = False
    print(json.dumps(line), flush=True)


def _profile_traffic(kernel, workload):
    """HBM bytes per launch from a committed copy-calibrated PMC summary
    (profiles/<kernel>_<workload>_traffic.json), or None."""
    tpath = os.path.join(ROOT, "profiles", f"{kernel}_{workload}_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    return None


C5_METRIC = ("C5 end-to-end decode tokens/s + resident KV bytes, random-init Llama-3-8B, batch 16, "
             "prompt 2048, 256 greedy steps")


def c5_model(device):
    from paged_tierkv_amd import workloads as W

    return W.llama3_8b_random(device)


def c5_generate(model, prompt, cache, steps, runtime=None):
    """Prefill, then `steps` greedy decode steps; returns (tokens [B, steps],
    decode seconds measured with a device sync on both sides, cache).  With
    ``runtime`` the decode steps go through hf_llama.DecodeGraphRunner
    (captured steps replayed as HIP graphs; the captures happen inside the
    timed region)."""
    import torch

    from paged_tierkv_amd import hf_llama

    toks = []
    with torch.no_grad():
        out = model(input_ids=prompt, past_key_values=cache, use_cache=True, logits_to_keep=1)
        cache = out.past_key_values
        tok = out.logits[:, -1].argmax(-1, keepdim=True)
        runner = hf_llama.DecodeGraphRunner(model, runtime) if runtime is not None else None
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            if runner is not None:
                logits = runner.step(tok)
            else:
                out = model(input_ids=tok, past_key_values=cache, use_cache=True, logits_to_keep=1)
                cache = out.past_key_values
                logits = out.logits
            tok = logits[:, -1].argmax(-1, keepdim=True)
            toks.append(tok)
        torch.cuda.synchronize()
        sec = time.perf_counter() - t0
    return torch.cat(toks, dim=1), sec, cache


def c5_forced(model, prompt, forced, cache, runtime=None):
    """Prefill, then feed forced[:, s] for every s (teacher forcing): the
    last-position logits of the prefill and of every step, fp16
    [steps + 1, B, V]."""
    import torch

    from paged_tierkv_amd import hf_llama

    outs = []
    with torch.no_grad():
        out = model(input_ids=prompt, past_key_values=cache, use_cache=True, logits_to_keep=1)
        outs.append(out.logits[:, -1].to(torch.float16, copy=True))
        cache = out.past_key_values
        runner = hf_llama.DecodeGraphRunner(model, runtime) if runtime is not None else None
        for s in range(forced.shape[1]):
            tok = forced[:, s: s + 1]
            if runner is not None:
                logits = runner.step(tok)
            else:
                out = model(input_ids=tok, past_key_values=cache, use_cache=True, logits_to_keep=1)
                cache = out.past_key_values
                logits = out.logits
            # A copy: the graph runner returns its static output buffer,
            # which a later replay overwrites.
            outs.append(logits[:, -1].to(torch.float16, copy=True))
    torch.cuda.synchronize()
    return torch.stack(outs)


def synced_step_ms(model, prompt, cache, steps):
    """Prefill, then `steps` greedy decode steps with a device sync after
    each; returns the wall time of every step in ms (the per-step view of
    c5_generate's run: which steps cost more, not the pipelined rate)."""
    import torch

    out_ms = []
    with torch.no_grad():
        out = model(input_ids=prompt, past_key_values=cache, use_cache=True, logits_to_keep=1)
        cache = out.past_key_values
        tok = out.logits[:, -1].argmax(-1, keepdim=True)
        torch.cuda.synchronize()
        for _ in range(steps):
            t0 = time.perf_counter()
            out = model(input_ids=tok, past_key_values=cache, use_cache=True, logits_to_keep=1)
            cache = out.past_key_values
            tok = out.logits[:, -1].argmax(-1, keepdim=True)
            torch.cuda.synchronize()
            out_ms.append((time.perf_counter() - t0) * 1e3)
    return out_ms


REF_METRIC = ("reference-API drop-in end-to-end decode tokens/s, TinyLlama-1.1B shape, batch 1, HOT+WARM, "
              "hot budget 8, policy every 64")
# The reference's own number for this setting (TierKV Triton path, HOT+WARM,
# hot budget 8, policy interval 64, TinyLlama-1.1B, ctx 512 / 1024 / 1536 /
# 1900) on one NVIDIA A10G: FINAL_EVALUATION_RESULTS.md:83-88.
REF_PUBLISHED_A10G = {512: 50.15, 1024: 49.22, 1536: 49.63, 1900: 46.51}


MICRO_METRIC = ("decode no-score / score latency ratio, the reference's kernel microbenchmark (kv 4, q 8, D 64, "
                "all-HOT dense pool, 4 / 16 / 64 blocks)")


def run_microbench(args, device):
    """benchmark_no_score_anomaly (tierkv_triton.py:504-673) through the
    drop-in: a dense ``TieredKVTensorPool`` whose HOT blocks are written with
    ``write_hot_tokens``, an identity block table, the reference's call, and
    its timing protocol -- 5 warm-up calls per path, then 50 calls each
    followed by a host synchronisation, wall clock -- for 4, 16 and 64
    blocks.  The no-score / score ratio is the reference's only kernel-level
    figure (0.73-0.86 on an A10G, main.py:3410-3412); its anomaly test is a
    ratio above 1.05.  Kernel-only times (one prepared launch per step,
    replayed from a HIP graph, HIP events) are reported beside it.  ``value`` is the ratio at
    64 blocks; a ratio near 1 means the score pass costs little."""
    import torch

    from paged_tierkv_amd import tierkv_policy as tp
    from paged_tierkv_amd.tierkv_hip import PreparedDecode, tierkv_decode_attention

    bs, kvh, qh, D = 16, 4, 8, 64
    gen = torch.Generator(device=device).manual_seed(5000)
    rows = []
    for nb in (4, 16, 64):
        mb = nb + 4
        pool = tp.TieredKVTensorPool(num_layers=1, block_size=bs, max_seq_len=mb * bs, max_blocks_per_layer=mb,
                                     pool_blocks=mb, pool_chunk_blocks=max(nb, 4))
        for phys in range(nb):
            k = torch.randn((1, kvh, bs, D), generator=gen, device=device, dtype=torch.float16)
            v = torch.randn((1, kvh, bs, D), generator=gen, device=device, dtype=torch.float16)
            pool.write_hot_tokens(phys, 0, k, v)
        table = torch.full((mb,), -1, device=device, dtype=torch.int32)
        table[:nb] = torch.arange(nb, device=device, dtype=torch.int32)
        states = torch.full((mb,), tp.HOT_STATE, device=device, dtype=torch.int32)
        kw = dict(query_states=torch.randn((1, qh, 1, D), generator=gen, device=device, dtype=torch.float16),
                  block_table=table, block_states=states, block_lengths=pool.block_lengths,
                  hot_k_pool=pool.hot_k_pool, hot_v_pool=pool.hot_v_pool, warm_k_pool=pool.warm_k_pool,
                  warm_v_pool=pool.warm_v_pool, k_scale=pool.k_scale, k_zero=pool.k_zero, v_scale=pool.v_scale,
                  v_zero=pool.v_zero, num_blocks=nb, num_key_value_groups=qh // kvh, scaling=D ** -0.5)
        for scores in (True, False):
            for _ in range(5):
                tierkv_decode_attention(**kw, return_scores=scores)
                torch.cuda.synchronize()
        _, with_sums = tierkv_decode_attention(**kw, return_scores=True)
        _, without = tierkv_decode_attention(**kw, return_scores=False)
        torch.cuda.synchronize()
        row = {"num_blocks": nb, "api_score_returns_tensor": with_sums is not None,
               "api_no_score_returns_none": without is None}
        for scores, key in ((True, "score"), (False, "no_score")):
            t0 = time.perf_counter()
            for _ in range(50):
                tierkv_decode_attention(**kw, return_scores=scores)
                torch.cuda.synchronize()
            row[f"t_{key}_ms"] = round((time.perf_counter() - t0) / 50 * 1e3, 4)
        for scores, key in ((True, "score"), (False, "no_score")):
            # kernel time: one prepared launch replayed from a HIP graph
            plan = PreparedDecode(**kw, return_scores=scores)
            sec, _ = graph_timed(lambda i: plan.launch(), 20, 400, 20)
            row[f"kernel_{key}_us"] = round(sec * 1e6, 3)
            del plan
        row["ratio_no_score_over_score"] = round(row["t_no_score_ms"] / row["t_score_ms"], 4)
        row["kernel_ratio_no_score_over_score"] = round(row["kernel_no_score_us"] / row["kernel_score_us"], 4)
        row["anomaly_present"] = row["ratio_no_score_over_score"] > 1.05
        log(f"[microbench] {nb:3d} blocks: no-score {row['t_no_score_ms']:.4f} ms, score {row['t_score_ms']:.4f} ms "
            f"(ratio {row['ratio_no_score_over_score']:.3f}); kernels {row['kernel_no_score_us']:.2f} / "
            f"{row['kernel_score_us']:.2f} us")
        rows.append(row)
        del pool, kw
    last = rows[-1]
    cfg = {"workload": "reference_microbench_no_score_anomaly", "kv_heads": kvh, "num_heads": qh, "head_dim": D,
           "block_size": bs, "block_counts": [4, 16, 64], "pool": "dense TieredKVTensorPool, all HOT",
           "timing": "per call: launch + host synchronise, wall clock, 50 calls (the reference's protocol)"}
    line = _line(MICRO_METRIC, last["ratio_no_score_over_score"], "ratio", 50, 5,
                 last["t_no_score_ms"] / 1e3, "f16", cfg, per_block_count=rows,
                 reference_ratio_a10g="0.73-0.86 (main.py:3410-3412)", roofline=None, cpu_baseline=None)
    print(json.dumps(line), flush=True)


def run_ref(args, device):
    """The reference's end-to-end setting through this build's drop-in for
    its Python API: a random-init TinyLlama-1.1B-shaped model (22 layers,
    hidden 2048, 32 / 4 heads, head_dim 64, FFN 5632, vocab 32000, fp16),
    batch 1, a uniform-random prompt, greedy decode through the HF hooks and
    the drop-in TieredKVRuntime (reference warm format, zero-logit COLD,
    HOT+WARM policy with hot budget 8, re-evaluated every 64 tokens).  Each
    decode step runs eagerly, as the reference's does.  Stock transformers
    with its dense DynamicCache on the same model and prompt is timed
    beside it."""
    import torch
    from transformers import DynamicCache, LlamaConfig, LlamaForCausalLM

    from paged_tierkv_amd import hf_llama, tierkv_policy as tp
    from paged_tierkv_amd.block_manager import BlockManager

    T, steps = args.ref_prompt, args.ref_steps
    cfg = LlamaConfig(hidden_size=2048, intermediate_size=5632, num_hidden_layers=22, num_attention_heads=32,
                      num_key_value_heads=4, head_dim=64, vocab_size=32000, max_position_embeddings=4096,
                      rope_theta=10000.0, initializer_range=0.02, rms_norm_eps=1e-5, tie_word_embeddings=False)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float16)
    try:
        with torch.device(device):
            model = LlamaForCausalLM(cfg).eval()
    finally:
        torch.set_default_dtype(prev)
    hf_llama.install()
    prompt = torch.randint(0, cfg.vocab_size, (1, T), generator=torch.Generator().manual_seed(2)).to(device)

    def runtime():
        tp.reset_global_tierkv()
        return tp.TieredKVRuntime(block_manager=BlockManager(total_blocks=8192), num_layers=cfg.num_hidden_layers,
                                  block_size=16, hot_budget=8, max_seq_len=T + steps + 16, attention_backend="triton",
                                  policy_interval=64, policy_mode="hot_warm")

    log(f"[ref] warm-up (kernels, GEMM heuristics) on {torch.cuda.get_device_name(0)}")
    c5_generate(model, prompt[:, :64], runtime().cache, 8)
    log(f"[ref] drop-in runtime: prompt {T}, {steps} greedy steps")
    rt = runtime()
    toks, sec, _ = c5_generate(model, prompt, rt.cache, steps)
    tps = steps / sec
    metrics = rt.collect_memory_metrics() if hasattr(rt, "collect_memory_metrics") else {}
    log(f"[ref] drop-in: {tps:.1f} tok/s ({sec / steps * 1e3:.2f} ms/step)")
    # Per-step view (a sync after every step): plain steps against the policy
    # steps (every 64th), beside the same view of stock dense.
    per_step = synced_step_ms(model, prompt, runtime().cache, steps)
    policy_idx = [i for i in range(steps) if (i + 1) % 64 == 0]
    plain = [t for i, t in enumerate(per_step) if i not in policy_idx and i > 0]
    synced = {"drop_in_plain_step_median_ms": round(statistics.median(plain), 3),
              "drop_in_policy_step_mean_ms": (round(statistics.mean(per_step[i] for i in policy_idx), 3)
                                              if policy_idx else None),
              "drop_in_first_step_ms": round(per_step[0], 3)}
    dense = None
    if not args.no_dense_baseline:
        c5_generate(model, prompt[:, :64], DynamicCache(config=cfg), 8)
        _, dsec, _ = c5_generate(model, prompt, DynamicCache(config=cfg), steps)
        dense = {"tokens_per_s": round(steps / dsec, 1), "ms_per_step": round(dsec / steps * 1e3, 3)}
        synced["dense_step_median_ms"] = round(statistics.median(synced_step_ms(model, prompt,
                                                                                 DynamicCache(config=cfg), steps)), 3)
        log(f"[ref] dense: {dense['tokens_per_s']} tok/s")
    log(f"[ref] synced steps: {synced}")
    hf_llama.uninstall()
    tp.reset_global_tierkv()
    pub = REF_PUBLISHED_A10G.get(T)
    line = _line(REF_METRIC, round(tps, 1), "tokens/s", steps, 8, sec / steps, "f16",
                 {"workload": "ref_tinyllama_b1_e2e", "batch": 1, "prompt": T, "decode_steps": steps,
                  "block_size": 16, "hot_budget": 8, "policy_interval": 64, "policy_mode": "hot_warm",
                  "warm_format": "reference uint8 per-token asymmetric", "cold": "zero_logit",
                  "runtime": "reference-API drop-in (tierkv_policy.TieredKVRuntime) through the HF hooks",
                  "decode_steps_as": "eager"},
                 dense_hf_baseline=dense, synced_steps=synced,
                 reference_published=({"tokens_per_s": pub, "hardware": "NVIDIA A10G",
                                       "source": "FINAL_EVALUATION_RESULTS.md:83-88"} if pub else None))
    line["data"] = "synthetic: random-init weights N(0, 0.02), uniform random prompt ids"
    line["ms_per_step"] = round(sec / steps * 1e3, 3)
    line["vs_baseline"] = round(tps / pub, 3) if pub else None
    if metrics:
        line["kv_metrics"] = {k: v for k, v in metrics.items() if isinstance(v, (int, float))}
    print(json.dumps(line), flush=True)


def run_c5(args, device):
    import torch
    from transformers import DynamicCache

    from paged_tierkv_amd import hf_llama
    from paged_tierkv_amd.runtime import BatchedTieredKVRuntime

    B, T, steps = args.c5_batch, args.c5_prompt, args.c5_steps
    log(f"[c5] building random-init Llama-3-8B on {torch.cuda.get_device_name(0)}")
    model = c5_model(device)
    cfg = model.config
    hf_llama.install()
    prompt = torch.randint(0, cfg.vocab_size, (B, T), generator=torch.Generator().manual_seed(1)).to(device)

    def runtime():
        return BatchedTieredKVRuntime(cfg.num_hidden_layers, B, cfg.num_key_value_heads, cfg.head_dim,
                                      T + steps + 16, block_size=16, hot_fraction=0.15, warm_fraction=0.55,
                                      policy_mode="hot_warm_cold", policy_interval=64, warm_format="absmax_i8",
                                      cold_mode="masked", device=device)

    log("[c5] warm-up run (kernels, GEMM heuristics)")
    c5_generate(model, prompt[:, :256], runtime().cache, 8)
    eager = None
    if not args.c5_eager:
        log(f"[c5] tiered run (eager steps): batch {B}, prompt {T}, {steps} greedy steps, policy every 64")
        rt = runtime()
        _, esec, _ = c5_generate(model, prompt, rt.cache, steps)
        rt.check_errors()
        eager = {"tokens_per_s": round(B * steps / esec, 1), "ms_per_step": round(esec / steps * 1e3, 3)}
        log(f"[c5] tiered eager: {eager['tokens_per_s']} tok/s ({eager['ms_per_step']} ms/step)")
        del rt
        torch.cuda.empty_cache()
    mode = "eager" if args.c5_eager else "HIP graphs"
    log(f"[c5] tiered run ({mode}): batch {B}, prompt {T}, {steps} greedy steps, policy every 64")
    rt = runtime()
    toks, sec, _ = c5_generate(model, prompt, rt.cache, steps, runtime=None if args.c5_eager else rt)
    rt.check_errors()
    metrics = rt.memory_metrics()
    tps = B * steps / sec
    log(f"[c5] tiered ({mode}): {tps:.1f} tok/s ({sec / steps * 1e3:.2f} ms/step), KV pools "
        f"{metrics['physical_pool_bytes'] / 2**20:.1f} MiB allocated ({metrics['resident_kv_bytes'] / 2**20:.1f} MiB "
        f"resident) vs dense {metrics['dense_equivalent_bytes'] / 2**20:.1f} MiB")
    dense = agreement = like_for_like = None
    if not args.no_dense_baseline:
        del rt
        torch.cuda.empty_cache()
        log("[c5] dense baseline: stock transformers DynamicCache, same model and prompt")
        c5_generate(model, prompt[:, :256], DynamicCache(config=cfg), 8)
        dtoks, dsec, dcache = c5_generate(model, prompt, DynamicCache(config=cfg), steps)
        kv_bytes = 0
        for layer in dcache.layers:
            for t in (layer.keys, layer.values):
                kv_bytes += t.numel() * t.element_size()
        del dcache
        dense = {"tokens_per_s": round(B * steps / dsec, 1), "ms_per_step": round(dsec / steps * 1e3, 3),
                 "kv_bytes": kv_bytes, "decode_steps_as": "eager (stock transformers)"}
        log(f"[c5] dense: {dense['tokens_per_s']} tok/s, KV {kv_bytes / 2**20:.1f} MiB")
        if eager is not None:
            like_for_like = {"tiered_eager_tokens_per_s": eager["tokens_per_s"],
                             "dense_eager_tokens_per_s": dense["tokens_per_s"],
                             "ratio": round(eager["tokens_per_s"] / dense["tokens_per_s"], 3)}
        # Output agreement (random-init logits are nearly flat, so greedy
        # tokens of a tiered run say nothing): every block HOT, teacher-forced
        # on the dense run's own greedy tokens, against the dense run's logits.
        n = min(steps, 32)
        torch.cuda.empty_cache()
        log(f"[c5] all-HOT tiered runtime teacher-forced on the dense run's first {n} tokens")
        dlog = c5_forced(model, prompt, dtoks[:, :n], DynamicCache(config=cfg))
        # The rounding floor of two correct fp16 attention implementations:
        # stock transformers' eager attention against its SDPA, same tokens.
        impl = cfg._attn_implementation
        cfg._attn_implementation = "eager"
        try:
            elog = c5_forced(model, prompt, dtoks[:, :n], DynamicCache(config=cfg))
        finally:
            cfg._attn_implementation = impl
        floor = (elog.float() - dlog.float()).abs()
        del elog
        hot_rt = BatchedTieredKVRuntime(cfg.num_hidden_layers, B, cfg.num_key_value_heads, cfg.head_dim,
                                        T + n + 16, block_size=16, hot_fraction=1.0, warm_fraction=0.0,
                                        policy_mode="hot_warm", policy_interval=64, device=device)
        hlog = c5_forced(model, prompt, dtoks[:, :n], hot_rt.cache, runtime=hot_rt)
        hot_rt.check_errors()
        err = (hlog.float() - dlog.float()).abs()
        agreement = {"steps": n, "max_abs_logit_err": round(err.max().item(), 5),
                     "mean_abs_logit_err": round(err.mean().item(), 6),
                     "logit_std": round(dlog.float().std().item(), 4),
                     "argmax_agreement": round((hlog.argmax(-1) == dlog.argmax(-1)).float().mean().item(), 4),
                     "floor_dense_eager_vs_sdpa": {"max_abs_logit_err": round(floor.max().item(), 5),
                                                   "mean_abs_logit_err": round(floor.mean().item(), 6)}}
        log(f"[c5] all-HOT vs dense (teacher-forced): {agreement}")
        del hot_rt, hlog, dlog
    hf_llama.uninstall()
    line = {
        "metric": C5_METRIC,
        "value": round(tps, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": 8,
        "ms_per_step": round(sec / steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: random-init weights N(0, 0.02), uniform random prompt ids",
        "config": {"workload": "c5_llama3_8b_e2e", "batch": B, "prompt": T, "decode_steps": steps,
                   "block_size": 16, "hot_fraction": 0.15, "warm_fraction": 0.55, "policy_interval": 64,
                   "policy_mode": "hot_warm_cold", "warm_format": "int8 absmax per (block, kv head)",
                   "cold": "masked", "attention": "tiered HIP decode kernel; prefill via the model's SDPA",
                   "decode_steps_as": mode},
        "tiered_eager_steps": eager,
        # Eager against eager: the HIP-graph figure above has no stock
        # counterpart (transformers' decode loop runs eagerly).
        "like_for_like_eager": like_for_like,
        "all_hot_vs_dense_teacher_forced": agreement,
        # Headline memory figure: the HBM the tiered pools hold (allocated,
        # free slots included) against the dense fp16 cache; the bytes of the
        # blocks resident at the end beside it.
        "kv_physical_pool_bytes": metrics["physical_pool_bytes"],
        "kv_dense_equivalent_bytes": metrics["dense_equivalent_bytes"],
        "kv_physical_compression_x": round(metrics["physical_compression_x"], 3),
        "kv_resident_bytes": metrics["resident_kv_bytes"],
        "kv_resident_compression_x": round(metrics["compression_x"], 3),
        "tiers_at_end": {k: metrics[k] for k in ("hot_blocks", "warm_blocks", "cold_blocks")},
        "dense_hf_baseline": dense,
    }
    print(json.dumps(line), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        log("bench.py measures one GPU: every box in this pool has one MI355X, so --gpus must be 1.")
        sys.exit(2)
    import torch

    device = torch.device("cuda:0")
    if args.mode == "copy":
        copy_calibration(device)
        return
    if args.mode == "ceiling":
        print(json.dumps(ceiling(device)), flush=True)
        return
    if args.workload == "c5":
        run_c5(args, device)
        return
    if args.workload == "c1":
        run_c1(args, device)
        return
    if args.workload == "prefill":
        run_prefill(args, device)
        return
    if args.workload == "ref":
        run_ref(args, device)
        return
    if args.workload == "microbench":
        run_microbench(args, device)
        return
    if args.workload in ("c2a", "promote"):
        run_c2a(args, device)
        return
    if args.workload == "c2b":
        run_c2b(args, device)
        return
    run_decode(args, device)


def run_decode(args, device):
    """C3 (default) / C4: one step = one decode-attention launch for one layer
    over the whole batch; ``--layers`` layer buffers rotate.

    Order: one launch per layer (code-object load), the box's HBM ceilings,
    at least 60 ms of untimed decode launches (``settle``; their count is in
    the line as ``untimed_settle_launches``), then W untimed warm-up steps
    and exactly K timed steps.  The clocks follow the load with a lag: after
    a few seconds idle C3 launches run 3-8 % slow for about 20 ms, and right
    after the ceiling measurement's streaming reads about 1 % slow for
    several milliseconds, which a short timed run (K = 20) would otherwise
    fall into; after the settle, K timed steps see the clocks a decode loop
    sees whatever K is.  Every launch is a
    ``PreparedDecode`` (validated and bound once: one C call per step, a few
    microseconds of host time), and the K timed launches are enqueued while
    the warm-up launches still run, so the timed region holds the K kernels
    back to back -- a host synchronisation between warm-up and timing would
    put the enqueue cost of the first timed call inside a short run's timed
    region.  Both sides of the run are bracketed by a device synchronisation."""
    import torch

    from paged_tierkv_amd import workloads as W
    from paged_tierkv_amd.tierkv_hip import PreparedDecode, workspace_error_word

    scores = bool(args.scores)
    fmt = args.warm_format
    log(f"[bench] building {args.layers} layers of {args.workload} ({fmt}, cold {args.cold}, scores {scores}) on "
        f"{torch.cuda.get_device_name(0)}")
    layers = build_layers(args, device)
    case = layers[0]["case"]
    nbytes = W.ideal_bytes(case.block_states, case.num_blocks, case.num_heads, case.kv_heads, case.head_dim,
                           warm_format=fmt, return_scores=scores)

    plans = [PreparedDecode(**L["args"], return_scores=scores, cold_mode=args.cold, splits=args.splits or None,
                            deterministic=args.deterministic) for L in layers]
    # Each layer's plan is launched once before the ceiling measurement: a
    # kernel's first launch in a process loads its code object (milliseconds
    # of host time, the GPU idle meanwhile).
    for plan in plans:
        plan.launch()
    # The box's own ceiling for this access pattern: the same bytes gathered
    # as shuffled 4 KB tiles with the decode kernel's load policy, no
    # arithmetic; and a streaming read.
    ceil = ceiling(device, c3_bytes=nbytes, stream_grids=(4096,), reps=400, release=False)
    settle_launches = settle(plans)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for i in range(args.warmup):
        plans[i % len(plans)].launch()
    h0 = time.perf_counter()
    e0.record()
    for i in range(args.steps):
        plans[(args.warmup + i) % len(plans)].launch()
    e1.record()
    host = (time.perf_counter() - h0) / max(args.steps, 1)
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) / 1e3 / args.steps
    assert workspace_error_word(device) == 0, "kernel flagged an out-of-range slot"
    ratio = None
    if scores:
        # The reference's only published kernel-level figure: no-score over
        # score latency of the decode launch, 0.73-0.86 on an A10G
        # (main.py:3410-3412).  The same layers without scores, timed the
        # same way right after (clocks already steady).
        plain = [PreparedDecode(**L["args"], return_scores=False, cold_mode=args.cold, splits=args.splits or None,
                                deterministic=args.deterministic) for L in layers]
        for i in range(max(args.warmup, len(plain))):
            plain[i % len(plain)].launch()
        f0, f1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        f0.record()
        for i in range(args.steps):
            plain[i % len(plain)].launch()
        f1.record()
        torch.cuda.synchronize()
        sec0 = f0.elapsed_time(f1) / 1e3 / args.steps
        ratio = {"no_score_us_per_layer_step": round(sec0 * 1e6, 3), "score_us_per_layer_step": round(sec * 1e6, 3),
                 "no_score_over_score": round(sec0 / sec, 4), "reference_a10g": "0.73-0.86"}
        log(f"[bench] no-score {sec0 * 1e6:.2f} us, score {sec * 1e6:.2f} us: ratio {sec0 / sec:.3f}")
    gbs = nbytes / sec / 1e9
    log(f"[bench] measured ceilings: gather {ceil['gather_4k_tiles_GBps']} GB/s, stream read "
        f"{ceil['stream_read_grid4096_GBps']} GB/s")
    log(f"[bench] {sec * 1e6:.2f} us/layer-step, {gbs:.1f} GB/s algorithmic ({gbs / PEAK_HBM_GBS:.1%} of peak); "
        f"host enqueue {host * 1e6:.1f} us per launch")

    # HBM bytes per launch of the decode kernel from the committed rocprofv3
    # FETCH_SIZE / WRITE_SIZE summary of this workload (copy-calibrated).
    traffic = None
    tag = _decode_tag(case.name, fmt, args.cold, scores, args.deterministic)
    # (the deterministic hand-out moves the same bytes: the default launch's profile)
    tpath = os.path.join(ROOT, "profiles", f"tiered_decode_kernel_{_decode_tag(case.name, fmt, args.cold, scores)}"
                                           "_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] timing the CPU baseline")

        def sample_bytes(nseq):
            return W.ideal_bytes(case.block_states[:nseq], case.num_blocks, case.num_heads, case.kv_heads,
                                 case.head_dim, warm_format=fmt)

        cpu = cpu_baseline(args, layers[0], sample_bytes)
    measured_ceiling = {"gather_4k_tiles_GBps": ceil["gather_4k_tiles_GBps"],
                        "stream_read_GBps": ceil["stream_read_grid4096_GBps"],
                        "frac_of_gather": round(gbs / ceil["gather_4k_tiles_GBps"], 4)}
    fmt_name = ("int8 absmax per (block, kv head)" if fmt == "absmax_i8"
                else "reference uint8 per-token asymmetric (fp16 scale + zero)")
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
        "config": {"workload": tag, "batch": case.batch, "num_heads": case.num_heads,
                   "kv_heads": case.kv_heads, "head_dim": case.head_dim, "block_size": case.block_size,
                   "blocks_per_seq": case.num_blocks, "tiers_per_seq": list(case.tier_counts()[0]),
                   "warm_format": fmt_name, "cold": args.cold, "return_scores": scores,
                   "deterministic": bool(args.deterministic), "layers_rotated": args.layers},
        "us_per_layer_step": round(sec * 1e6, 3),
        "tokens_per_s_32_layers": round(case.batch / (32 * sec), 1),
        "ideal_bytes_per_step": nbytes,
        "host_enqueue_us_per_launch": round(host * 1e6, 2),
        "untimed_settle_launches": settle_launches,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic},
        "measured_ceiling": measured_ceiling,
        "cpu_baseline": cpu,
    }
    if ratio is not None:
        line["score_path"] = ratio
    if (args.workload == "c3" and fmt == "absmax_i8" and args.cold == "masked" and not scores and not args.splits
            and not args.no_extras and not args.deterministic):
        del plans, layers
        torch.cuda.empty_cache()
        line["extra_decode_figures"] = extra_decode_figures(args, device, sec)
    print(json.dumps(line), flush=True)


def extra_decode_figures(args, device, c3_sec):
    """The other decode lines of the scope, timed right after the headline C3
    line and the same way (prepared launches, ``--layers`` rotated buffers,
    warm-up, then exactly ``--steps`` launches between HIP events): C3 with
    score sums (the policy step's launch) and its no-score/score ratio, C3 in
    the reference WARM format with zero-logit COLD (the drop-in's default),
    C4 with and without score sums (each with its own profile summary under
    profiles/), and C3 with the deterministic tile hand-out and its time
    over the default launch's."""
    import argparse

    import torch

    from paged_tierkv_amd import workloads as W
    from paged_tierkv_amd.tierkv_hip import PreparedDecode, workspace_error_word

    def timed(workload, fmt, cold, scores, det=False):
        a = argparse.Namespace(**vars(args))
        a.workload, a.warm_format, a.cold, a.scores = workload, fmt, cold, scores
        layers = build_layers(a, device)
        case = layers[0]["case"]
        nbytes = W.ideal_bytes(case.block_states, case.num_blocks, case.num_heads, case.kv_heads, case.head_dim,
                               warm_format=fmt, return_scores=scores)
        plans = [PreparedDecode(**L["args"], return_scores=scores, cold_mode=cold, deterministic=det) for L in layers]
        # Building the inputs leaves the GPU idle long enough for its clocks
        # to drop: keep it launching for >= 60 ms before the timed launches.
        settle(plans, at_least=max(args.warmup, 4 * len(plans)))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(args.steps):
            plans[i % len(plans)].launch()
        e1.record()
        torch.cuda.synchronize()
        assert workspace_error_word(device) == 0, "kernel flagged an out-of-range slot"
        sec = e0.elapsed_time(e1) / 1e3 / args.steps
        del plans, layers
        torch.cuda.empty_cache()
        gbs = nbytes / sec / 1e9
        out = {"workload": _decode_tag(case.name, fmt, cold, scores, det), "us_per_layer_step": round(sec * 1e6, 3),
               "achieved_GBps": round(gbs, 2), "frac": round(gbs / PEAK_HBM_GBS, 4), "ideal_bytes_per_step": nbytes}
        log(f"[bench] extra {out['workload']}: {out['us_per_layer_step']} us, {gbs / PEAK_HBM_GBS:.1%} of peak")
        return out, sec

    res = {}
    c3s, sec = timed("c3", "absmax_i8", "masked", True)
    c3s["no_score_over_score"] = round(c3_sec / sec, 4)
    res["c3_scores"] = c3s
    res["c3_ref_u8_zero_logit"], _ = timed("c3", "ref_u8", "zero_logit", False)
    res["c4"], c4_sec = timed("c4", "absmax_i8", "masked", False)
    c4s, sec = timed("c4", "absmax_i8", "masked", True)
    c4s["no_score_over_score"] = round(c4_sec / sec, 4)
    res["c4_scores"] = c4s
    c3d, sec = timed("c3", "absmax_i8", "masked", False, True)
    c3d["over_default"] = round(sec / c3_sec, 4)
    res["c3_deterministic"] = c3d
    res["reference_no_score_over_score_a10g"] = "0.73-0.86"
    return res


def _decode_tag(name, fmt, cold, scores, det=False):
    """Workload name of a decode bench line (and of its profile files)."""
    tag = name
    if fmt != "absmax_i8":
        tag += "_ref_u8"
    if cold != "masked":
        tag += "_" + cold
    if scores:
        tag += "_scores"
    if det:
        tag += "_deterministic"
    return tag


if __name__ == "__main__":
    main()

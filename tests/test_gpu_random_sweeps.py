"""Seeded random sweeps against the oracle, beyond the fixed shapes of the
other GPU tests:

* demotion in both WARM formats, and promotion of the demoted slots, over
  random geometry (kv heads 1-8, block
  sizes 1-64, head dims including ones the one-wave kernels do not take),
  job counts, lengths (0 included), the zero-padded tail or not, and value
  mixes chosen to reach the codec's edges: exact ties, subnormals, constant
  rows, all-positive rows (negative zero points) and magnitudes near the
  fp16 maximum (a row whose range overflows to infinity takes the IEEE
  path).  Codes, scales, zero points and the promoted fp16 values bit for
  bit (quantize_fp16_to_int8 / dequantize_int8_to_fp16,
  tierkv_policy.py:21-44; BASELINE's absmax codec);
* block mass from probabilities (bit for bit) and tier labels (exactly) over
  random shapes, block sizes, lengths, budgets, modes and score ties
  (compute_block_scores, tierkv_policy.py:1380-1389; enforce_budget /
  enforce_tiered_budget, 1391-1477);
* the batched runtime over random scenarios (batch, kv heads, group, head
  dim, prompt length from one token, steps, tick interval, budgets, policy
  mode, WARM format, COLD mode): tables, states, lengths and pool contents
  equal to oracle.runtime after the prefill and after every step, decode
  outputs within BASELINE's tolerance (the runtime generalises
  TieredKVRuntime, tierkv_policy.py:1534-1912, to a batch);
* prefill block scores over random batch, GQA group (1-8), prompt length,
  head dim, block size, dtype and logit scale, at 1e-4 relative to the
  float64 oracle (compute_block_scores on the eager prefill attention,
  tierkv_policy.py:1380-1389).

The seeds are fixed, so every run draws the same cases."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import codec
from oracle import policy as opolicy
from oracle.policy import prefill_block_mass as oracle_prefill_mass
from oracle.runtime import BatchedRuntimeOracle
from paged_tierkv_amd import kernels
from paged_tierkv_amd.runtime import BatchedTieredKVRuntime

from helpers import assert_close
from test_gpu_runtime import _compare, _oracle_out

pytestmark = pytest.mark.gpu


def _eq(a, b, what):
    a = np.asarray(a)
    b = np.asarray(b)
    assert a.shape == b.shape, f"{what}: shape {a.shape} != {b.shape}"
    if a.dtype in (np.float16, np.float32):
        a = a.view(np.uint16 if a.dtype == np.float16 else np.uint32)
        b = b.view(a.dtype)
    assert np.array_equal(a, b), f"{what}: {int((a != b).sum())} of {a.size} differ"


def _values(rng, shape):
    kind = int(rng.integers(0, 6))
    if kind == 0:
        v = rng.standard_normal(shape) * rng.uniform(0.01, 8)
    elif kind == 1:
        v = rng.standard_normal(shape) * 1000
    elif kind == 2:
        v = rng.integers(-3, 4, shape) * 2.0 ** int(rng.integers(-24, 4))
    elif kind == 3:
        v = np.abs(rng.standard_normal(shape)) + rng.uniform(0, 100)
    elif kind == 4:
        v = rng.uniform(-65504, 65504, shape)
    else:
        v = np.full(shape, float(rng.standard_normal()))
    return np.clip(v, -65504, 65504).astype(np.float16)


# Rows near the fp16 maximum overflow the oracle's fp16 range on purpose (an
# infinite scale then dequantizes a zero offset to NaN, in both).
@pytest.mark.filterwarnings("ignore:overflow encountered in cast:RuntimeWarning")
@pytest.mark.filterwarnings("ignore:invalid value encountered in multiply:RuntimeWarning")
@pytest.mark.parametrize("seed", [3, 7])
def test_demotion_random_geometry_bit_exact(device, seed):
    rng = np.random.default_rng(seed)
    for it in range(40):
        heads = int(rng.integers(1, 9))
        bs = int(rng.choice([1, 2, 4, 8, 16, 32, 64]))
        dim = int(rng.choice([8, 12, 16, 24, 32, 40, 48, 64, 96, 128, 192, 256]))
        tiles = int(rng.integers(1, 40))
        slots = tiles + int(rng.integers(0, 5))
        n = int(rng.integers(1, tiles + 1))
        fmt = str(rng.choice(["ref_u8", "absmax_i8"]))
        pad = bool(rng.random() < 0.5)
        src_k = _values(rng, (tiles, heads, bs, dim))
        src_v = _values(rng, (tiles, heads, bs, dim))
        jobs = rng.permutation(tiles)[:n].astype(np.int32)
        dst = rng.permutation(slots)[:n].astype(np.int32)
        lens = rng.integers(0, bs + 1, n).astype(np.int32)
        print(f"[sweep] demote seed={seed} it={it} fmt={fmt} heads={heads} bs={bs} dim={dim} n={n} pad={pad}",
              flush=True)
        wdt = torch.uint8 if fmt == "ref_u8" else torch.int8
        warm_k = torch.full((slots, heads, bs, dim), 77, dtype=wdt, device=device)
        warm_v = warm_k.clone()
        if fmt == "ref_u8":
            ks = torch.full((slots, heads, bs, 1), -1.0, dtype=torch.float16, device=device)
            kz, vs, vz = ks.clone(), ks.clone(), ks.clone()
        else:
            ks = torch.full((slots, heads), -1.0, device=device)
            vs, kz, vz = ks.clone(), None, None
        kernels.demote_to_warm(torch.from_numpy(src_k).to(device), torch.from_numpy(src_v).to(device),
                               torch.from_numpy(jobs), torch.from_numpy(dst), torch.from_numpy(lens),
                               warm_k, warm_v, ks, kz, vs, vz, warm_format=fmt, pad_tail=pad)
        torch.cuda.synchronize()
        for i in range(n):
            s, d, ln = int(jobs[i]), int(dst[i]), int(lens[i])
            if ln == 0:
                continue
            for nm, src, codes, sc, zp in (("k", src_k, warm_k, ks, kz), ("v", src_v, warm_v, vs, vz)):
                what = f"{nm} it={it} job={i}"
                if fmt == "ref_u8":
                    q, scale, z = codec.quantize_ref_u8(src[s, :, :ln])
                    _eq(codes[d, :, :ln].cpu().numpy(), q, f"codes {what}")
                    _eq(sc[d, :, :ln].cpu().numpy(), scale, f"scale {what}")
                    _eq(zp[d, :, :ln].cpu().numpy(), z, f"zero point {what}")
                else:
                    q, scale = codec.quantize_absmax_i8(src[s, :, :ln])
                    _eq(codes[d, :, :ln].cpu().numpy(), q, f"codes {what}")
                    _eq(sc[d].cpu().numpy(), scale, f"scale {what}")
        # Promotion of the same slots back to fp16 into fresh HOT slots:
        # dequantize_int8_to_fp16 (tierkv_policy.py:39-44) of the stored codes,
        # or fp16(code * scale) for absmax; tokens past a job's length untouched.
        hot_k = torch.full((n, heads, bs, dim), 9.0, dtype=torch.float16, device=device)
        hot_v = hot_k.clone()
        kernels.promote_to_hot(warm_k, warm_v, ks, kz, vs, vz, torch.from_numpy(dst),
                               torch.arange(n, dtype=torch.int32), torch.from_numpy(lens), hot_k, hot_v,
                               warm_format=fmt)
        torch.cuda.synchronize()
        for i in range(n):
            d, ln = int(dst[i]), int(lens[i])
            for nm, codes, sc, zp, hot in (("k", warm_k, ks, kz, hot_k), ("v", warm_v, vs, vz, hot_v)):
                c = codes[d, :, :ln].cpu().numpy()
                if fmt == "ref_u8":
                    exp = codec.dequantize_ref_u8(c, sc[d, :, :ln].cpu().numpy(), zp[d, :, :ln].cpu().numpy())
                else:
                    exp = (c.astype(np.float32) * sc[d].cpu().numpy()[:, None, None]).astype(np.float16)
                _eq(hot[i, :, :ln].cpu().numpy(), exp, f"promote {nm} it={it} job={i}")
                assert (hot[i, :, ln:].cpu() == 9.0).all(), f"promote {nm} it={it} job={i}: tail written"


@pytest.mark.parametrize("seed", [1, 11])
def test_block_mass_and_labels_random_shapes(device, seed):
    rng = np.random.default_rng(seed)
    for it in range(40):
        bs = int(rng.choice([1, 2, 4, 8, 16, 32, 64]))
        nblk = int(rng.integers(1, 300))
        b, h = int(rng.integers(1, 9)), int(rng.integers(1, 100))
        if b * h * nblk * bs <= 4_000_000:
            logits = rng.standard_normal((b, h, nblk * bs)) * rng.uniform(0.1, 4)
            probs = np.exp(logits - logits.max(-1, keepdims=True))
            probs = (probs / probs.sum(-1, keepdims=True)).astype(np.float32)
            lens = rng.integers(0, bs + 1, (b, nblk)).astype(np.int32) if rng.random() < 0.5 else None
            print(f"[sweep] mass seed={seed} it={it} b={b} h={h} blocks={nblk} bs={bs}", flush=True)
            exp = opolicy.block_mass_from_probs(probs, bs, lens)
            got = kernels.block_mass_from_probs(torch.from_numpy(probs).to(device), bs,
                                                None if lens is None else torch.from_numpy(lens).to(device))
            _eq(got.cpu().numpy(), exp, f"block mass it={it}")
        n = int(rng.integers(1, 8193))
        bb = int(rng.integers(1, 6))
        kind = int(rng.integers(0, 3))
        if kind == 0:
            scores = rng.standard_normal((bb, n)).astype(np.float32)
        elif kind == 1:
            scores = (rng.integers(0, 5, (bb, n)) * 0.25).astype(np.float32)     # many exact ties
        else:
            scores = np.where(rng.random((bb, n)) < 0.5, 0.0, -0.0).astype(np.float32)   # 0.0 ties -0.0
        cur = rng.integers(0, 3, (bb, n)).astype(np.int32)
        hot, warm = int(rng.integers(0, n + 3)), int(rng.integers(0, n + 3))
        mode = str(rng.choice(["hot_warm", "hot_warm_cold", "hot_only"]))
        demoted = int(rng.choice([1, 2]))
        print(f"[sweep] labels seed={seed} it={it} b={bb} n={n} hot={hot} warm={warm} mode={mode}", flush=True)
        exp = opolicy.tier_labels(scores, cur, hot, warm, mode, demoted_state=demoted)
        got = kernels.tier_labels(torch.from_numpy(scores).to(device), torch.from_numpy(cur).to(device), hot, warm,
                                  mode, demoted_state=demoted)
        assert np.array_equal(got.cpu().numpy(), exp), f"labels it={it} n={n} hot={hot} warm={warm} mode={mode}"


def test_batched_runtime_random_scenarios(device):
    rng = np.random.default_rng(5)
    for sc in range(8):
        B = int(rng.integers(1, 7))
        kv = int(rng.choice([1, 2, 4]))
        G = int(rng.choice([1, 2, 4, 8]))
        D = int(rng.choice([64, 128]))
        bs = 16
        prompt, steps, interval = int(rng.integers(1, 600)), int(rng.integers(5, 70)), int(rng.integers(1, 17))
        policy_mode = str(rng.choice(["hot_warm_cold", "hot_warm"]))
        warm_format = str(rng.choice(["absmax_i8", "ref_u8"]))
        cold_mode = str(rng.choice(["masked", "zero_logit"]))
        hot_f = float(rng.uniform(0.05, 0.6))
        warm_f = float(rng.uniform(0.0, 1.0 - hot_f))
        print(f"[sweep] runtime sc={sc} B={B} kv={kv} G={G} D={D} prompt={prompt} steps={steps} "
              f"interval={interval} mode={policy_mode} fmt={warm_format} cold={cold_mode}", flush=True)
        gen = torch.Generator().manual_seed(int(rng.integers(0, 2 ** 31)))
        rt = BatchedTieredKVRuntime(1, B, kv, D, prompt + steps + 16, block_size=bs, hot_fraction=hot_f,
                                    warm_fraction=warm_f, policy_mode=policy_mode, policy_interval=interval,
                                    warm_format=warm_format, cold_mode=cold_mode, device=device)
        orc = BatchedRuntimeOracle(B, kv, D, bs, rt.max_blocks, rt.hot_slots, rt.warm_slots, policy_mode,
                                   warm_format)
        k = torch.randn((B, kv, prompt, D), generator=gen).half()
        v = torch.randn((B, kv, prompt, D), generator=gen).half()
        n0 = -(-prompt // bs)
        scores = torch.rand((B, n0), generator=gen)
        rt.prefill_layer(0, k.to(device), v.to(device), block_scores=scores)
        hot_b, warm_b = rt.budgets(n0)
        orc.prefill(k.numpy(), v.numpy(), scores.numpy(), hot_b, warm_b)
        torch.cuda.synchronize()
        _compare(rt, orc, f"sc={sc} prefill")
        scaling = D ** -0.5
        for step in range(steps):
            tick = rt.begin_step()
            q = torch.randn((B, kv * G, 1, D), generator=gen).half()
            k1 = torch.randn((B, kv, 1, D), generator=gen).half()
            v1 = torch.randn((B, kv, 1, D), generator=gen).half()
            out = rt.decode_layer(0, q.to(device), k1.to(device), v1.to(device), G, scaling, policy_step=tick)
            orc.append(k1.numpy(), v1.numpy())
            exp = _oracle_out(rt, orc, q[:, :, 0].numpy(), G, scaling, cold_mode)
            assert_close(out[:, 0].float().cpu().numpy(), exp, what=f"sc={sc} step {step} output")
            if tick:
                hb, wb = rt.budgets(int(orc.nb.max()))
                orc.tick(rt.last_score_sums.cpu().numpy(), hb, wb)
            rt.end_step()
            torch.cuda.synchronize()
            _compare(rt, orc, f"sc={sc} step {step}{' (tick)' if tick else ''}")
        rt.check_errors()
        del rt
        torch.cuda.empty_cache()


def test_prefill_block_mass_random_shapes(device):
    rng = np.random.default_rng(2)
    for it in range(12):
        hkv = int(rng.choice([1, 2, 4, 8]))
        g_ = int(rng.integers(1, 9))
        b, t = int(rng.integers(1, 4)), int(rng.integers(1, 700))
        d, bs = int(rng.choice([64, 128])), int(rng.choice([16, 32, 64]))
        dtype = torch.float16 if rng.random() < 0.7 else torch.bfloat16
        sc = float(rng.uniform(0.3, 3.0))
        print(f"[sweep] prefill it={it} B={b} H={hkv * g_} Hkv={hkv} T={t} D={d} bs={bs} {dtype} scale={sc:.2f}",
              flush=True)
        gen = torch.Generator().manual_seed(100 + it)
        q = (torch.randn((b, hkv * g_, t, d), generator=gen) * sc).to(dtype)
        k = (torch.randn((b, hkv, t, d), generator=gen) * sc).to(dtype)
        got = kernels.prefill_block_mass(q.to(device), k.to(device), bs, d ** -0.5).cpu().numpy()
        want = oracle_prefill_mass(q.float().numpy(), k.float().numpy(), d ** -0.5, bs)
        np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-9, err_msg=f"prefill it={it}")

"""GPU parity of the demotion (quantize) and promotion (dequantize) kernels:
codes, scales, zero points and table rewrites bit-exact against the oracle
codec, which is itself pinned to golden vectors written by the reference's
quantize_fp16_to_int8 (tierkv_policy.py:21-36)."""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import codec
from paged_tierkv_amd import kernels, workloads as W

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _eq(a, b, what):
    a = np.asarray(a)
    b = np.asarray(b)
    assert a.shape == b.shape, f"{what}: shape {a.shape} != {b.shape}"
    if a.dtype in (np.float16, np.float32):
        a = a.view(np.uint16 if a.dtype == np.float16 else np.uint32)
        b = b.view(a.dtype)
    bad = a != b
    assert not bad.any(), f"{what}: {int(bad.sum())} of {a.size} differ; first {np.argwhere(bad)[:3].tolist()}"


@pytest.mark.parametrize("bs,dim", [(16, 128), (16, 64), (4, 16), (8, 12), (32, 128), (16, 256), (64, 128)])
def test_absmax_demote_bit_exact(device, bs, dim):
    print(f"[quant] absmax bs={bs} dim={dim}", flush=True)
    g = torch.Generator().manual_seed(bs * 100 + dim)
    tiles, heads = 23, 3
    src_k = (torch.randn((tiles, heads, bs, dim), generator=g) * 2).half()
    src_v = torch.randn((tiles, heads, bs, dim), generator=g).half()
    src_k[5] = 0                                        # zero tile -> scale 0, codes 0
    jobs = torch.tensor([3, 5, 0, 22, 11, 7], dtype=torch.int32)
    dst = torch.tensor([4, 0, 9, 2, 7, 1], dtype=torch.int32)
    lens = torch.tensor([bs, bs, 1, bs - 1, bs, 2], dtype=torch.int32)
    warm_k = torch.full((10, heads, bs, dim), 77, dtype=torch.int8, device=device)
    warm_v = warm_k.clone()
    ks = torch.full((10, heads), -1.0, device=device)
    vs = ks.clone()
    table = torch.full((2, 8), -1, dtype=torch.int32, device=device)
    states = torch.zeros((2, 8), dtype=torch.int32, device=device)
    pos = torch.tensor([0, 3, 8, 15, -1, 9], dtype=torch.int32)
    kernels.demote_to_warm(src_k.to(device), src_v.to(device), jobs, dst, lens, warm_k, warm_v, ks, None, vs, None,
                           warm_format="absmax_i8", block_table=table, block_states=states, table_pos=pos)
    torch.cuda.synchronize()
    for i in range(len(jobs)):
        s, d, n = int(jobs[i]), int(dst[i]), int(lens[i])
        for name, src, codes, sc in (("k", src_k, warm_k, ks), ("v", src_v, warm_v, vs)):
            q, scale = codec.quantize_absmax_i8(src[s, :, :n].numpy())
            _eq(codes[d, :, :n].cpu().numpy(), q, f"{name} codes job {i}")
            _eq(sc[d].cpu().numpy(), scale, f"{name} scale job {i}")
            assert int(codes[d, :, n:].abs().sum()) == 0, "tail codes must be 0"
    t = table.view(-1).cpu().numpy()
    st = states.view(-1).cpu().numpy()
    for i, p in enumerate(pos.tolist()):
        if p >= 0:
            assert t[p] == int(dst[i]) and st[p] == 1
    assert (t[[1, 2, 4]] == -1).all()


def test_absmax_demote_half_integer_quotients(device):
    """Tiles whose absmax is 127 * 2^j have the exact scale 2^j, so every
    element (k + 0.5) * 2^j has the quotient k + 0.5 exactly: rintf's
    half-to-even ties, which the kernel's reciprocal fast path must hand to
    the IEEE division.  Mixed with tiles of near-tie quotients from random
    scales."""
    g = torch.Generator().manual_seed(7)
    tiles, heads, bs, dim = 12, 8, 16, 128
    k = torch.randint(-127, 127, (tiles, heads, bs, dim), generator=g).double()
    j = torch.randint(-12, 3, (tiles, heads, 1, 1), generator=g).double()
    x = (k + 0.5) * torch.pow(2.0, j)
    x[..., 0, 0] = 127 * torch.pow(2.0, j[..., 0, 0])
    x = x.half()
    x[tiles // 2:] = (torch.randn((tiles - tiles // 2, heads, bs, dim), generator=g) * 3).half()
    idx = torch.arange(tiles, dtype=torch.int32)
    warm = torch.empty((tiles, heads, bs, dim), dtype=torch.int8, device=device)
    warm_v = torch.empty_like(warm)
    ks = torch.empty((tiles, heads), device=device)
    vs = torch.empty_like(ks)
    xd = x.to(device)
    kernels.demote_to_warm(xd, xd, idx, idx, torch.full((tiles,), bs, dtype=torch.int32), warm, warm_v,
                           ks, None, vs, None, warm_format="absmax_i8")
    torch.cuda.synchronize()
    q, scale = codec.quantize_absmax_i8(x.numpy())
    _eq(warm.cpu().numpy(), q, "half-integer quotient codes")
    _eq(warm_v.cpu().numpy(), q, "half-integer quotient codes (V)")
    _eq(ks.cpu().numpy(), scale, "half-integer quotient scales")
    ties = np.abs(np.abs(x[: tiles // 2].float().numpy() / scale[: tiles // 2, :, None, None]) % 1 - 0.5) == 0
    assert ties.sum() == (tiles // 2) * heads * (bs * dim - 1), "every element but the absmax is an exact tie"


def test_c2a_demotion_full_size_bit_exact(device):
    case = W.config2a()
    print(f"[quant] C2(a) demote {len(case.demote_logical)} of {case.hot_k.shape[0]} blocks", flush=True)
    n = len(case.demote_logical)
    warm_k = torch.empty((n, 8, 16, 128), dtype=torch.int8, device=device)
    warm_v = torch.empty_like(warm_k)
    ks = torch.empty((n, 8), device=device)
    vs = torch.empty_like(ks)
    table = case.table.to(device)
    states = case.states.to(device)
    src = case.table[0, case.demote_logical]
    kernels.demote_to_warm(case.hot_k.to(device), case.hot_v.to(device), src, case.warm_slots,
                           torch.full((n,), 16, dtype=torch.int32), warm_k, warm_v, ks, None, vs, None,
                           warm_format="absmax_i8", block_table=table, block_states=states,
                           table_pos=case.demote_logical.to(torch.int32))
    torch.cuda.synchronize()
    qk, sk = codec.quantize_absmax_i8(case.hot_k[src.long()].numpy())
    qv, sv = codec.quantize_absmax_i8(case.hot_v[src.long()].numpy())
    _eq(warm_k.cpu().numpy(), qk, "C2a K codes")
    _eq(warm_v.cpu().numpy(), qv, "C2a V codes")
    _eq(ks.cpu().numpy(), sk, "C2a K scales")
    _eq(vs.cpu().numpy(), sv, "C2a V scales")
    exp_table = case.table.clone()
    exp_states = case.states.clone()
    exp_table[0, case.demote_logical] = case.warm_slots
    exp_states[0, case.demote_logical] = 1
    _eq(table.cpu().numpy(), exp_table.numpy(), "C2a table")
    _eq(states.cpu().numpy(), exp_states.numpy(), "C2a states")


def test_reference_codec_demote_matches_golden(device):
    g = np.load(os.path.join(GOLDEN, "codec_ref_u8.npz"))
    x = torch.from_numpy(g["x"])                      # [7, 4, 16, 64] fp16
    tiles, heads, bs, dim = x.shape
    idx = torch.arange(tiles, dtype=torch.int32)
    warm_k = torch.zeros((tiles, heads, bs, dim), dtype=torch.uint8, device=device)
    warm_v = warm_k.clone()
    sc = lambda: torch.zeros((tiles, heads, bs, 1), dtype=torch.float16, device=device)
    ks, kz, vs, vz = sc(), sc(), sc(), sc()
    xd = x.to(device)
    kernels.demote_to_warm(xd, xd, idx, idx, torch.full((tiles,), bs, dtype=torch.int32), warm_k, warm_v,
                           ks, kz, vs, vz, warm_format="ref_u8")
    torch.cuda.synchronize()
    _eq(warm_k.cpu().numpy(), g["q"], "codes vs reference golden")
    _eq(ks.cpu().numpy(), g["scale"], "scale vs reference golden")
    _eq(kz.cpu().numpy(), g["zero"], "zero vs reference golden")
    # promotion back to fp16 == dequantize_int8_to_fp16 of the golden codes
    hot = torch.zeros((tiles, heads, bs, dim), dtype=torch.float16, device=device)
    hot_v = hot.clone()
    kernels.promote_to_hot(warm_k, warm_v, ks, kz, vs, vz, idx, idx, torch.full((tiles,), bs, dtype=torch.int32),
                           hot, hot_v, warm_format="ref_u8")
    torch.cuda.synchronize()
    _eq(hot.cpu().numpy(), g["deq"], "promote vs reference dequant golden")


# (16, 64), (16, 128), (32, 128), (8, 256): the one-wave-per-tile kernels
# (head_dim / 8 lanes per token row); (16, 12), (64, 128): the per-workgroup
# fallback kernels (head_dim not a multiple of 8, tile above 512 vectors).
@pytest.mark.parametrize("bs,dim", [(16, 64), (16, 128), (32, 128), (8, 256), (16, 12), (64, 128)])
@pytest.mark.parametrize("pad_tail", [False, True])
def test_reference_codec_partial_blocks(device, pad_tail, bs, dim):
    print(f"[quant] ref_u8 partial blocks bs={bs} dim={dim} pad_tail={pad_tail}", flush=True)
    g = torch.Generator().manual_seed(9)
    heads = 2
    src = (torch.randn((4, heads, bs, dim), generator=g) * 3).half()
    src[3, 1, 0] = 0.5                                       # constant row: scale 0 -> 1
    lens = torch.tensor([bs, 5, 1, min(9, bs)], dtype=torch.int32)
    idx = torch.arange(4, dtype=torch.int32)
    dst = torch.tensor([2, 0, 3, 1], dtype=torch.int32)
    warm = torch.full((4, heads, bs, dim), 200, dtype=torch.uint8, device=device)
    warm_v = warm.clone()
    ks = torch.full((4, heads, bs, 1), 7.0, dtype=torch.float16, device=device)
    kz, vs, vz = ks.clone(), ks.clone(), ks.clone()
    src_v = (src * -2).contiguous()
    kernels.demote_to_warm(src.to(device), src_v.to(device), idx, dst, lens, warm, warm_v, ks, kz, vs, vz,
                           warm_format="ref_u8", pad_tail=pad_tail)
    torch.cuda.synchronize()
    for i in range(4):
        n, d = int(lens[i]), int(dst[i])
        for what, x, wc, sc, zc in (("K", src, warm, ks, kz), ("V", src_v, warm_v, vs, vz)):
            q, s, z = codec.quantize_ref_u8(x[i, :, :n].numpy())
            _eq(wc[d, :, :n].cpu().numpy(), q, f"{what} codes {i}")
            _eq(sc[d, :, :n].cpu().numpy(), s, f"{what} scale {i}")
            _eq(zc[d, :, :n].cpu().numpy(), z, f"{what} zero {i}")
            tail_codes = wc[d, :, n:].cpu().numpy()
            if pad_tail:   # write_warm_block (tierkv_policy.py:989-995)
                assert (tail_codes == 0).all() and (sc[d, :, n:].cpu().numpy() == 1).all()
                assert (zc[d, :, n:].cpu().numpy() == 0).all()
            else:          # compact demote_to_warm leaves the tail untouched
                assert (tail_codes == 200).all() and (sc[d, :, n:].cpu().numpy() == 7).all()
    # Promotion back (dequantize_int8_to_fp16, tierkv_policy.py:39-44) of the
    # first lengths[i] tokens; the HOT tail stays untouched.
    hot = torch.full((5, heads, bs, dim), 9.0, dtype=torch.float16, device=device)
    hot_v = hot.clone()
    pdst = torch.tensor([4, 1, 0, 2], dtype=torch.int32)
    kernels.promote_to_hot(warm, warm_v, ks, kz, vs, vz, dst, pdst, lens, hot, hot_v, warm_format="ref_u8")
    torch.cuda.synchronize()
    for i in range(4):
        n, d, h = int(lens[i]), int(dst[i]), int(pdst[i])
        for what, wc, sc, zc, out in (("K", warm, ks, kz, hot), ("V", warm_v, vs, vz, hot_v)):
            exp = codec.dequantize_ref_u8(wc[d, :, :n].cpu().numpy(), sc[d, :, :n].cpu().numpy(),
                                          zc[d, :, :n].cpu().numpy())
            _eq(out[h, :, :n].cpu().numpy(), exp, f"{what} promote {i}")
            assert (out[h, :, n:].cpu() == 9.0).all()
    assert (hot[3].cpu() == 9.0).all()


@pytest.mark.parametrize("dim", [128, 64, 12])
def test_reference_codec_special_rows(device, dim):
    """Rows that exercise every branch of the reference codec's arithmetic:
    constant rows (scale 0 -> 1), a range that overflows fp16 (scale +inf,
    the IEEE-division path), large offsets (quotients in the thousands,
    where fp16 spacing is 2-4), subnormal fp16 values and ordinary rows.
    head_dim 128 / 64 run the one-wave-per-tile kernel, 12 the fallback."""
    print(f"[quant] ref_u8 special rows dim={dim}", flush=True)
    g = torch.Generator().manual_seed(21)
    heads, bs = 2, 16
    x = torch.randn((6, heads, bs, dim), generator=g) * 3
    x[1, 0] = 0.5
    x[1, 1] = 0.0
    x[2] = torch.where(torch.arange(dim) % 2 == 0, 40000.0, -40000.0) + torch.randn((heads, bs, dim), generator=g)
    x[3] = 10.0 + torch.randn((heads, bs, dim), generator=g) * 0.1
    x[4] = torch.randn((heads, bs, dim), generator=g) * 1e-4
    x[5, :, ::2] = -7.25
    x = x.half()
    n = x.shape[0]
    idx = torch.arange(n, dtype=torch.int32)
    warm = torch.zeros((n, heads, bs, dim), dtype=torch.uint8, device=device)
    warm_v = warm.clone()
    meta = [torch.zeros((n, heads, bs, 1), dtype=torch.float16, device=device) for _ in range(4)]
    xd = x.to(device)
    kernels.demote_to_warm(xd, xd, idx, idx, torch.full((n,), bs, dtype=torch.int32), warm, warm_v, *meta,
                           warm_format="ref_u8")
    torch.cuda.synchronize()
    with np.errstate(all="ignore"):
        q, sc, zp = codec.quantize_ref_u8(x.numpy())
    _eq(warm.cpu().numpy(), q, "special rows codes")
    _eq(warm_v.cpu().numpy(), q, "special rows V codes")
    _eq(meta[0].cpu().numpy(), sc, "special rows scales")
    _eq(meta[1].cpu().numpy(), zp, "special rows zero points")
    assert np.isinf(sc[2].astype(np.float32)).all()          # the overflow tile took the IEEE path


def test_c2_reference_codec_round_trip_bit_exact(device):
    """C2's pool in the reference's WARM format: 512 of the demoted blocks
    quantized, table rewritten, then promoted into fresh HOT slots."""
    case = W.config2a()
    n = 512
    logical = case.demote_logical[:n]
    print(f"[quant] C2 ref_u8 demote + promote of {n} blocks", flush=True)
    src = case.table[0, logical]
    slots = torch.randperm(n, generator=torch.Generator().manual_seed(5)).to(torch.int32)
    warm_k = torch.empty((n, 8, 16, 128), dtype=torch.uint8, device=device)
    warm_v = torch.empty_like(warm_k)
    meta = [torch.empty((n, 8, 16, 1), dtype=torch.float16, device=device) for _ in range(4)]
    table, states = case.table.to(device), case.states.to(device)
    kernels.demote_to_warm(case.hot_k.to(device), case.hot_v.to(device), src, slots,
                           torch.full((n,), 16, dtype=torch.int32), warm_k, warm_v, *meta,
                           warm_format="ref_u8", block_table=table, block_states=states,
                           table_pos=logical.to(torch.int32))
    torch.cuda.synchronize()
    for what, x, wc, sc, zc in (("K", case.hot_k, warm_k, meta[0], meta[1]), ("V", case.hot_v, warm_v, meta[2], meta[3])):
        q, s, z = codec.quantize_ref_u8(x[src.long()].numpy())
        _eq(wc.cpu()[slots.long()].numpy(), q, f"C2 ref {what} codes")
        _eq(sc.cpu()[slots.long()].numpy(), s, f"C2 ref {what} scales")
        _eq(zc.cpu()[slots.long()].numpy(), z, f"C2 ref {what} zeros")
    exp_table, exp_states = case.table.clone(), case.states.clone()
    exp_table[0, logical] = slots
    exp_states[0, logical] = 1
    _eq(table.cpu().numpy(), exp_table.numpy(), "C2 ref table")
    _eq(states.cpu().numpy(), exp_states.numpy(), "C2 ref states")
    hot_k = torch.empty((n, 8, 16, 128), dtype=torch.float16, device=device)
    hot_v = torch.empty_like(hot_k)
    kernels.promote_to_hot(warm_k, warm_v, *meta, slots, torch.arange(n, dtype=torch.int32),
                           torch.full((n,), 16, dtype=torch.int32), hot_k, hot_v, warm_format="ref_u8",
                           block_table=table, block_states=states, table_pos=logical.to(torch.int32))
    torch.cuda.synchronize()
    for what, wc, sc, zc, out in (("K", warm_k, meta[0], meta[1], hot_k), ("V", warm_v, meta[2], meta[3], hot_v)):
        exp = codec.dequantize_ref_u8(wc.cpu()[slots.long()].numpy(), sc.cpu()[slots.long()].numpy(),
                                      zc.cpu()[slots.long()].numpy())
        _eq(out.cpu().numpy(), exp, f"C2 ref {what} promote")
    exp_table[0, logical] = torch.arange(n, dtype=torch.int32)
    exp_states[0, logical] = 0
    _eq(table.cpu().numpy(), exp_table.numpy(), "C2 promote table")
    _eq(states.cpu().numpy(), exp_states.numpy(), "C2 promote states")


@pytest.mark.parametrize("dim", [128, 64])
def test_reference_codec_every_scale(device, dim):
    """One token row per positive finite fp16 maximum M (row minimum 0, so
    the row's scale is fp16(M / 255)): the quotients of every reachable
    scale go through the per-row reciprocal (hardware reciprocal plus a
    Newton step) and the FMA correction on the GPU itself; codes, scales and
    zero points must equal the oracle's bit for bit."""
    print(f"[quant] ref_u8 every scale dim={dim}", flush=True)
    m = np.arange(1, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)   # every positive finite fp16
    rows = int(np.ceil(m.size / 32)) * 32                                            # whole [2 heads, 16 tokens] tiles
    m = np.concatenate([m, np.ones(rows - m.size, np.float32)])
    u = np.random.default_rng(31).random((rows, dim), dtype=np.float32)
    x = (m[:, None] * u).astype(np.float16)
    x[:, 0] = 0.0
    x[:, 1] = m.astype(np.float16)
    x = torch.from_numpy(x.reshape(rows // 32, 2, 16, dim))
    n = x.shape[0]
    idx = torch.arange(n, dtype=torch.int32)
    warm = torch.zeros((n, 2, 16, dim), dtype=torch.uint8, device=device)
    meta = [torch.zeros((n, 2, 16, 1), dtype=torch.float16, device=device) for _ in range(4)]
    xd = x.to(device)
    kernels.demote_to_warm(xd, xd, idx, idx, torch.full((n,), 16, dtype=torch.int32), warm, warm.clone(), *meta,
                           warm_format="ref_u8")
    torch.cuda.synchronize()
    q, sc, zp = codec.quantize_ref_u8(x.numpy())
    assert len(np.unique(sc)) > 20000                     # most fp16 scale values are reached
    _eq(meta[0].cpu().numpy(), sc, "every-scale scales")
    _eq(meta[1].cpu().numpy(), zp, "every-scale zero points")
    _eq(warm.cpu().numpy(), q, "every-scale codes")

def test_absmax_promote_bit_exact(device):
    g = torch.Generator().manual_seed(4)
    codes = torch.randint(-127, 128, (5, 2, 16, 128), generator=g, dtype=torch.int8)
    scales = torch.rand((5, 2), generator=g) * 0.1
    lens = torch.tensor([16, 3, 16, 7, 1], dtype=torch.int32)
    src = torch.tensor([4, 0, 2, 1, 3], dtype=torch.int32)
    dst = torch.tensor([0, 1, 2, 3, 4], dtype=torch.int32)
    hot = torch.full((5, 2, 16, 128), 9.0, dtype=torch.float16, device=device)
    hot_v = hot.clone()
    cd = codes.to(device)
    sd = scales.to(device)
    table = torch.zeros(16, dtype=torch.int32, device=device)
    states = torch.ones(16, dtype=torch.int32, device=device)
    kernels.promote_to_hot(cd, cd, sd, None, sd, None, src, dst, lens, hot, hot_v, warm_format="absmax_i8",
                           block_table=table, block_states=states, table_pos=[1, 2, 3, 4, 5])
    torch.cuda.synchronize()
    for i in range(5):
        n = int(lens[i])
        exp = (codes[int(src[i]), :, :n].float() * scales[int(src[i])][:, None, None]).half()
        _eq(hot[i, :, :n].cpu().numpy(), exp.numpy(), f"promote {i}")
        assert (hot[i, :, n:].cpu() == 9.0).all()
    assert table[1:6].tolist() == [0, 1, 2, 3, 4] and states[1:6].tolist() == [0] * 5

"""GPU parity of the batched tiered runtime (paged_tierkv_amd.runtime)
against its CPU model (oracle.runtime): prefill into HOT / WARM / COLD,
per-step appends across block boundaries, and device-side policy ticks.

Bit-exact: slot tables, states, lengths, block counts, HOT contents and WARM
codes / scales of every live block (the allocation order is fixed).  The
tick ranks the decode kernel's own probability sums on both sides, so the
label decisions are compared on identical inputs.  Attention outputs: the
BASELINE tolerance (2e-3 abs, 1e-2 rel) against the oracle decode over the
oracle's pools."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.decode import decode_attention as oracle_decode
from oracle.runtime import BatchedRuntimeOracle
from paged_tierkv_amd.runtime import BatchedTieredKVRuntime

from helpers import assert_close

pytestmark = pytest.mark.gpu


def _compare(rt: BatchedTieredKVRuntime, orc: BatchedRuntimeOracle, what: str) -> None:
    st = rt.layers[0]
    nb = st.nblocks.cpu().numpy()
    np.testing.assert_array_equal(nb, orc.nb, err_msg=f"{what}: block counts")
    n = int(nb.max())
    tab, sts, lns = (x.cpu().numpy()[:, :n] for x in (st.table, st.states, st.lengths))
    np.testing.assert_array_equal(sts, orc.states[:, :n], err_msg=f"{what}: states")
    np.testing.assert_array_equal(lns, orc.lengths[:, :n], err_msg=f"{what}: lengths")
    np.testing.assert_array_equal(tab, orc.table[:, :n], err_msg=f"{what}: slots")
    hk, hv = st.hot_k.cpu().numpy(), st.hot_v.cpu().numpy()
    wk, wv = st.warm_k.cpu().numpy(), st.warm_v.cpu().numpy()
    ks, vs = st.k_scale.cpu().numpy(), st.v_scale.cpu().numpy()
    for b in range(rt.batch):
        for i in range(n):
            slot, s, ln = int(tab[b, i]), int(sts[b, i]), int(lns[b, i])
            if s == 0:
                np.testing.assert_array_equal(hk[slot, :, :ln], orc.hot_k[slot, :, :ln], err_msg=f"{what}: HOT K {b},{i}")
                np.testing.assert_array_equal(hv[slot, :, :ln], orc.hot_v[slot, :, :ln], err_msg=f"{what}: HOT V {b},{i}")
            elif s == 1:
                np.testing.assert_array_equal(wk[slot, :, :ln], orc.warm_k[slot, :, :ln], err_msg=f"{what}: WARM K {b},{i}")
                np.testing.assert_array_equal(wv[slot, :, :ln], orc.warm_v[slot, :, :ln], err_msg=f"{what}: WARM V {b},{i}")
                if rt.warm_format == "absmax_i8":
                    np.testing.assert_array_equal(ks[slot], orc.k_scale[slot], err_msg=f"{what}: k scale {b},{i}")
                    np.testing.assert_array_equal(vs[slot], orc.v_scale[slot], err_msg=f"{what}: v scale {b},{i}")
                else:
                    np.testing.assert_array_equal(ks[slot, :, :ln], orc.k_scale[slot, :, :ln])
                    np.testing.assert_array_equal(st.k_zero.cpu().numpy()[slot, :, :ln], orc.k_zero[slot, :, :ln])
                    np.testing.assert_array_equal(vs[slot, :, :ln], orc.v_scale[slot, :, :ln])
                    np.testing.assert_array_equal(st.v_zero.cpu().numpy()[slot, :, :ln], orc.v_zero[slot, :, :ln])


def _oracle_out(rt, orc, q, groups, scaling, cold_mode):
    n = int(orc.nb.max())
    args = [orc.hot_k, orc.hot_v, orc.warm_k, orc.warm_v, orc.k_scale, getattr(orc, "k_zero", None),
            orc.v_scale, getattr(orc, "v_zero", None)]
    return oracle_decode(q, orc.table, orc.states, orc.lengths, orc.nb, *args, groups, scaling,
                         warm_format=rt.warm_format, cold_mode=cold_mode)


@pytest.mark.parametrize("warm_format,policy_mode,cold_mode", [
    ("absmax_i8", "hot_warm_cold", "masked"),
    ("ref_u8", "hot_warm_cold", "zero_logit"),
    ("absmax_i8", "hot_warm", "masked"),
])
def test_batched_runtime_matches_model(device, warm_format, policy_mode, cold_mode):
    print(f"[runtime] fmt={warm_format} mode={policy_mode} cold={cold_mode}", flush=True)
    B, kv, G, D, bs = 4, 2, 4, 128, 16
    prompt, steps, interval = 16 * 20 + 5, 48, 8
    # Budgets small enough that the hot_warm_cold ticks must evict (the
    # resident count outgrows hot + warm as blocks are appended).
    hot_f, warm_f = (0.25, 0.15) if policy_mode == "hot_warm_cold" else (0.2, 0.5)
    gen = torch.Generator().manual_seed(7)
    rt = BatchedTieredKVRuntime(1, B, kv, D, prompt + steps + 16, block_size=bs, hot_fraction=hot_f,
                                warm_fraction=warm_f, policy_mode=policy_mode, policy_interval=interval,
                                warm_format=warm_format, cold_mode=cold_mode, device=device)
    orc = BatchedRuntimeOracle(B, kv, D, bs, rt.max_blocks, rt.hot_slots, rt.warm_slots, policy_mode, warm_format)
    k = torch.randn((B, kv, prompt, D), generator=gen).half()
    v = torch.randn((B, kv, prompt, D), generator=gen).half()
    n0 = -(-prompt // bs)
    scores = torch.rand((B, n0), generator=gen)
    scores[:, 3] = scores[:, 4]        # a tie: the lower index ranks first
    rt.prefill_layer(0, k.to(device), v.to(device), block_scores=scores)
    hot_b, warm_b = rt.budgets(n0)
    orc.prefill(k.numpy(), v.numpy(), scores.numpy(), hot_b, warm_b)
    torch.cuda.synchronize()
    _compare(rt, orc, "prefill")
    scaling = D ** -0.5
    for step in range(steps):
        tick = rt.begin_step()
        q = torch.randn((B, kv * G, 1, D), generator=gen).half()
        k1 = torch.randn((B, kv, 1, D), generator=gen).half()
        v1 = torch.randn((B, kv, 1, D), generator=gen).half()
        out = rt.decode_layer(0, q.to(device), k1.to(device), v1.to(device), G, scaling, policy_step=tick)
        orc.append(k1.numpy(), v1.numpy())
        exp = _oracle_out(rt, orc, q[:, :, 0].numpy(), G, scaling, cold_mode)
        assert_close(out[:, 0].float().cpu().numpy(), exp, what=f"step {step} output")
        if tick:
            n = int(orc.nb.max())
            hb, wb = rt.budgets(n)
            orc.tick(rt.last_score_sums.cpu().numpy(), hb, wb)
        rt.end_step()
        torch.cuda.synchronize()
        _compare(rt, orc, f"step {step}{' (tick)' if tick else ''}")
    rt.check_errors()
    # The ticks did move blocks between tiers (the comparison above is not
    # vacuous), and promotions landed in HOT slots their own tick freed (the
    # demotion data moves first).
    assert orc.migrations["demote"] > 0 and orc.migrations["promote"] > 0, orc.migrations
    assert orc.migrations["promote_into_freed"] > 0, orc.migrations
    if policy_mode == "hot_warm_cold":
        assert orc.migrations["evict"] > 0, orc.migrations
    m = rt.memory_metrics()
    assert m["hot_blocks"] + m["warm_blocks"] + m["cold_blocks"] == int(orc.nb.sum())
    # Device telemetry counters equal the counts of the model's tables.
    want = []
    for tier in (0, 1, 2):
        mask = np.zeros_like(orc.states, dtype=bool)
        for b in range(B):
            mask[b, :orc.nb[b]] = orc.states[b, :orc.nb[b]] == tier
        want.append((int(mask.sum()), int(orc.lengths[mask].sum())))
    got = rt.tier_counters().cpu().tolist()
    assert got == [w[0] for w in want] + [w[1] for w in want]
    assert 0 < m["resident_kv_bytes"] < m["dense_equivalent_bytes"]


def test_batched_runtime_reports_exhausted_slots(device):
    # A tiny HOT pool: the append that needs a slot it cannot get appends
    # nothing and raises through check_errors; nothing is overwritten.
    B, kv, D, bs = 2, 1, 64, 16
    rt = BatchedTieredKVRuntime(1, B, kv, D, 64, block_size=bs, hot_fraction=1.0, warm_fraction=0.0,
                                policy_mode="hot_warm", policy_interval=1000, device=device)
    k = torch.zeros((B, kv, rt.max_blocks * bs, D), dtype=torch.float16, device=device)
    rt.prefill_layer(0, k, k, block_scores=None)
    with pytest.raises(RuntimeError, match="table row is full"):
        one = torch.zeros((B, kv, 1, D), dtype=torch.float16, device=device)
        q = torch.zeros((B, kv, 1, D), dtype=torch.float16, device=device)
        rt.begin_step()
        rt.decode_layer(0, q, one, one, 1, D ** -0.5)
        rt.check_errors()


def test_fused_rope_append_is_bit_exact(device):
    """decode_layer(rope=(cos, sin)) rotates k into the pool and q for the
    kernel with transformers' own fp16 op order: pools, tables and the rotated
    query equal apply_rotary_pos_emb followed by the plain append, bit for
    bit, with HF's strided projection views as inputs."""
    transformers = pytest.importorskip("transformers")
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding, apply_rotary_pos_emb

    B, kv, G, D, bs, prompt = 3, 2, 4, 128, 16, 40
    H = kv * G
    cfg = LlamaConfig(hidden_size=H * D, num_attention_heads=H, num_key_value_heads=kv, head_dim=D,
                      max_position_embeddings=4096, rope_theta=500000.0)
    rot = LlamaRotaryEmbedding(cfg, device=device)
    gen = torch.Generator().manual_seed(21)
    k0 = torch.randn((B, kv, prompt, D), generator=gen).half().to(device)
    v0 = torch.randn((B, kv, prompt, D), generator=gen).half().to(device)
    rts = [BatchedTieredKVRuntime(1, B, kv, D, prompt + 64, block_size=bs, hot_fraction=1.0, warm_fraction=0.0,
                                  policy_mode="hot_warm", policy_interval=1000, device=device) for _ in range(2)]
    for rt in rts:
        rt.prefill_layer(0, k0, v0)
    for step in range(20):
        pos = torch.full((1, 1), prompt + step, dtype=torch.long, device=device)
        # HF's layout: projections [B, 1, heads * D] viewed as [B, heads, 1, D].
        qp = (torch.randn((B, 1, H * D), generator=gen) * 2).half().to(device).view(B, 1, H, D).transpose(1, 2)
        kp = (torch.randn((B, 1, kv * D), generator=gen) * 2).half().to(device).view(B, 1, kv, D).transpose(1, 2)
        vp = torch.randn((B, 1, kv * D), generator=gen).half().to(device).view(B, 1, kv, D).transpose(1, 2)
        cos, sin = rot(qp, pos)
        q_ref, k_ref = apply_rotary_pos_emb(qp, kp, cos, sin)
        out_ref = rts[0].decode_layer(0, q_ref, k_ref, vp, G, D ** -0.5)
        out = rts[1].decode_layer(0, qp, kp, vp, G, D ** -0.5, rope=(cos, sin))
        torch.testing.assert_close(out.float(), out_ref.float(), atol=2e-3, rtol=1e-2)
        for rt in rts:
            rt.end_step()
    a, b = rts[0].layers[0], rts[1].layers[0]
    for name in ("table", "states", "lengths", "nblocks", "open", "hot_k", "hot_v"):
        assert torch.equal(getattr(a, name), getattr(b, name)), name
    # The rotated query itself: run the fused append once more and compare.
    pos = torch.full((1, 1), prompt + 20, dtype=torch.long, device=device)
    qp = torch.randn((B, 1, H * D), generator=gen).half().to(device).view(B, 1, H, D).transpose(1, 2)
    cos, sin = rot(qp, pos)
    q_ref, _ = apply_rotary_pos_emb(qp, qp[:, :kv], cos, sin)
    q_rot = torch.empty((B, H, 1, D), dtype=torch.float16, device=device)
    st = b
    from paged_tierkv_amd import _lib
    lib = _lib.lib()
    kx = torch.zeros((B, kv, 1, D), dtype=torch.float16, device=device)
    rc = lib.tierkv_runtime_append_rope(
        _lib.ptr(qp), qp.stride(0), qp.stride(1), qp.stride(2), H, _lib.ptr(q_rot),
        _lib.ptr(kx), kx.stride(0), kx.stride(1), kx.stride(2), _lib.ptr(kx), kx.stride(0), kx.stride(1), kx.stride(2),
        _lib.ptr(cos), _lib.ptr(sin), 0, cos.stride(1), 1,
        _lib.ptr(st.table), _lib.ptr(st.states), _lib.ptr(st.lengths), rts[1].max_blocks, _lib.ptr(st.nblocks),
        _lib.ptr(st.open), B, 0, _lib.ptr(st.hot_k), _lib.ptr(st.hot_v), rts[1].hot_slots, _lib.ptr(st.hot_free),
        _lib.ptr(st.ctl), kv, bs, D, _lib.stream_of(device))
    _lib.check(rc)
    assert torch.equal(q_rot, q_ref.contiguous())

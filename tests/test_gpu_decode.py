"""GPU parity of the tiered decode-attention kernels against the CPU oracle
(oracle.decode restates _eager_reference_decode, tierkv_triton.py:708-820).

Tolerance: BASELINE's 2e-3 absolute / 1e-2 relative vs the fp32 reference
for outputs; the same for per-block probability sums."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from paged_tierkv_amd import workloads as W
from paged_tierkv_amd.tierkv_hip import tierkv_decode_attention, workspace_error_word

from helpers import assert_close, oracle_decode, oracle_warm, report, to_gpu_inputs

pytestmark = pytest.mark.gpu


def _run(case, fmt, device, cold_mode=None, return_scores=False, query_dtype=torch.float16, **kw):
    warm = oracle_warm(case, fmt)
    args = to_gpu_inputs(case, warm, device, query_dtype)
    out, scores = tierkv_decode_attention(**args, return_scores=return_scores,
                                          cold_mode=cold_mode or case.cold_mode, **kw)
    torch.cuda.synchronize()
    return warm, out, scores


def _check(case, fmt, device, cold_mode=None, return_scores=False, seqs=None, query_dtype=torch.float16, **kw):
    print(f"[decode] case={case.name} fmt={fmt} cold={cold_mode or case.cold_mode} scores={return_scores} "
          f"dtype={query_dtype} kw={kw}", flush=True)
    warm, out, scores = _run(case, fmt, device, cold_mode, return_scores, query_dtype, **kw)
    seqs = list(range(case.batch)) if seqs is None else seqs
    res = oracle_decode(case, warm, fmt, cold_mode, return_scores, seqs=seqs)
    exp_out, exp_sc = (res if return_scores else (res, None))
    got = out[seqs, 0].float().cpu().numpy()
    report(f"{case.name} {fmt} output ({len(seqs)} seqs)", assert_close(got, exp_out, what=f"{case.name} output"))
    if return_scores:
        sc = scores.cpu().numpy()
        if sc.ndim == 2:
            sc = sc[None]
        report(f"{case.name} {fmt} score_sums", assert_close(sc[seqs], exp_sc, what=f"{case.name} score_sums"))
    assert workspace_error_word(device) == 0
    return out, scores


# -- BASELINE configs -------------------------------------------------------

def test_c1_absmax_masked(device):
    _check(W.config1(), "absmax_i8", device, return_scores=True)


def test_c1_reference_format_zero_logit(device):
    _check(W.config1(), "ref_u8", device, cold_mode="zero_logit", return_scores=True)


def test_c1_bf16_query(device):
    case = W.config1()
    case.query = case.query.to(torch.bfloat16).to(torch.float16)   # the oracle sees the bf16 values
    _check(case, "absmax_i8", device, query_dtype=torch.bfloat16)


def test_c3_llama3_full(device):
    # Every one of the 32 sequences against the oracle.
    _check(W.config3(), "absmax_i8", device)


def test_c3_scores_full(device):
    _check(W.config3(), "absmax_i8", device, return_scores=True)


def test_c3_reference_format_zero_logit(device):
    # The drop-in's default WARM format (uint8 per-token codes) and COLD
    # semantics (zero logit) at C3's full size.
    _check(W.config3(), "ref_u8", device, cold_mode="zero_logit", return_scores=True)


def test_c4_long_context_full(device):
    _check(W.config4(), "absmax_i8", device, return_scores=True)


def _gqa16_long_case():
    # GQA 16 (four-wave workgroups), rows long enough that three splits stage
    # their statistics in the workspace (STAGE_GLOBAL) and eight in LDS.
    return W.make_tiered_case("gqa16_long", 2, 32, 2, 128, 1500, 150, 700, seed=77)


@pytest.mark.parametrize("which,fmt,cold,splits_seq,budgets", [
    ("c3", "absmax_i8", "masked", (None, None, 2, 3, None), (26, 154)),
    ("c3", "ref_u8", "zero_logit", (None, 2, 3, None), (26, 154)),
    # C4: one split (workspace stage + finalisation kernel) against five and
    # eight splits (list stage, finalised by each unit's last workgroup).
    ("c4", "absmax_i8", "masked", (None, 1, 5, 8, None), (102, 922)),
    ("c4", "ref_u8", "zero_logit", (None, 1, 5, 8), (102, 922)),
    ("gqa16", "absmax_i8", "zero_logit", (3, 4, 8, None, 3), (150, 700)),
])
def test_scores_reproducible(device, which, fmt, cold, splits_seq, budgets):
    """Score sums (and the labels ranked from them) are the same bits on every
    launch over the same inputs, whatever the split count, the stage (LDS
    block, LDS list, workspace) and the order in which waves met the tiles;
    the reference's score pass is a fixed sequential loop
    (tierkv_triton.py:121-145).  The first launch is also checked against
    the oracle."""
    from paged_tierkv_amd import kernels

    case = {"c3": W.config3, "c4": W.config4, "gqa16": _gqa16_long_case}[which]()
    print(f"[scores-repro] case={case.name} fmt={fmt} cold={cold} splits={splits_seq}", flush=True)
    warm = oracle_warm(case, fmt)
    args = to_gpu_inputs(case, warm, device)
    runs = []
    for splits in splits_seq:
        _, sc = tierkv_decode_attention(**args, return_scores=True, cold_mode=cold, splits=splits)
        scores = kernels.block_scores_from_sums(sc, args["block_lengths"], case.num_blocks)
        labels = kernels.tier_labels(scores, args["block_states"], budgets[0], budgets[1], mode="hot_warm_cold")
        torch.cuda.synchronize()
        runs.append((sc.cpu(), labels.cpu()))
    assert workspace_error_word(device) == 0
    seqs = list(range(min(case.batch, 4)))
    _, exp_sc = oracle_decode(case, warm, fmt, cold, True, seqs=seqs)
    sc0 = runs[0][0].numpy()
    report(f"{case.name} {fmt} {cold} score_sums", assert_close(sc0[seqs], exp_sc, what=f"{case.name} score_sums"))
    for (sc, lab), splits in zip(runs[1:], splits_seq[1:]):
        assert torch.equal(sc.view(torch.int32), runs[0][0].view(torch.int32)), f"score bits differ at splits={splits}"
        assert torch.equal(lab, runs[0][1]), f"labels differ at splits={splits}"


@pytest.mark.parametrize("which,fmt,cold,scores,splits", [
    ("c3", "absmax_i8", "masked", False, None),
    ("c3", "ref_u8", "zero_logit", True, None),
    ("c4", "absmax_i8", "masked", True, None),       # eight splits per unit: list stage, split merge
    ("gqa16", "ref_u8", "zero_logit", True, 3),      # four-wave workgroups, workspace stage
    ("c1", "absmax_i8", "masked", False, None),      # D = 64, many splits of a short row
])
def test_deterministic_launches_are_bit_identical(device, which, fmt, cold, scores, splits):
    """deterministic=True (TIERKV_DECODE_DETERMINISTIC) fixes each wave's share
    of the tiles, so the attention output is the same bits on every launch,
    as the reference's Triton kernel's is (tierkv_triton.py:45-145); the
    output stays within tolerance of the oracle, and the score sums equal the
    default launch's bit for bit."""
    case = {"c1": W.config1, "c3": W.config3, "c4": W.config4, "gqa16": _gqa16_long_case}[which]()
    print(f"[deterministic] case={case.name} fmt={fmt} cold={cold} scores={scores} splits={splits}", flush=True)
    warm = oracle_warm(case, fmt)
    args = to_gpu_inputs(case, warm, device)
    runs = []
    for _ in range(4):
        out, sc = tierkv_decode_attention(**args, return_scores=scores, cold_mode=cold, splits=splits,
                                          deterministic=True)
        torch.cuda.synchronize()
        runs.append((out.clone(), None if sc is None else sc.clone()))
    _, sc_default = tierkv_decode_attention(**args, return_scores=scores, cold_mode=cold, splits=splits)
    torch.cuda.synchronize()
    assert workspace_error_word(device) == 0
    for out, sc in runs[1:]:
        assert torch.equal(out.view(torch.int16), runs[0][0].view(torch.int16)), "output bits differ between launches"
        if scores:
            assert torch.equal(sc.view(torch.int32), runs[0][1].view(torch.int32))
    if scores:
        assert torch.equal(runs[0][1].view(torch.int32), sc_default.view(torch.int32)), \
            "score sums differ from the default launch's"
    seqs = list(range(min(case.batch, 8)))
    res = oracle_decode(case, warm, fmt, cold, scores, seqs=seqs)
    exp_out = res[0] if scores else res
    got = runs[0][0][seqs, 0].float().cpu().numpy()
    report(f"{case.name} {fmt} deterministic output", assert_close(got, exp_out, what=f"{case.name} output"))


def test_deterministic_flag_from_environment(device, monkeypatch):
    """TIERKV_DETERMINISTIC=1 makes deterministic launches the default, also
    for repeated calls that reuse their bound arguments."""
    case = W.config3(batch=8)
    warm = oracle_warm(case, "absmax_i8")
    args = to_gpu_inputs(case, warm, device)
    monkeypatch.setenv("TIERKV_DETERMINISTIC", "1")
    outs = []
    for _ in range(3):
        out, _ = tierkv_decode_attention(**args, cold_mode="masked")
        torch.cuda.synchronize()
        outs.append(out.clone())
    ref, _ = tierkv_decode_attention(**args, cold_mode="masked", deterministic=True, splits=None)
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o.view(torch.int16), ref.view(torch.int16))


def test_two_streams_concurrent(device):
    """Decodes of different shapes in flight on two streams at once: each
    stream has its own implicit workspace (split partials, arrival counters,
    score stage), so neither disturbs the other."""
    a = W.make_tiered_case("stream_a", 4, 32, 8, 128, 300, 30, 170, seed=61)
    b = W.make_tiered_case("stream_b", 3, 16, 4, 64, 200, 20, 120, seed=62)
    wa, wb = oracle_warm(a, "absmax_i8"), oracle_warm(b, "ref_u8")
    ia, ib = to_gpu_inputs(a, wa, device), to_gpu_inputs(b, wb, device)
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(device), torch.cuda.Stream(device)
    outs_a, outs_b = [], []
    for _ in range(12):
        with torch.cuda.stream(sa):
            outs_a.append(tierkv_decode_attention(**ia, return_scores=True, cold_mode="masked", splits=4))
        with torch.cuda.stream(sb):
            outs_b.append(tierkv_decode_attention(**ib, return_scores=True, cold_mode="zero_logit", splits=3))
    torch.cuda.synchronize()
    ea, esa = oracle_decode(a, wa, "absmax_i8", "masked", True)
    eb, esb = oracle_decode(b, wb, "ref_u8", "zero_logit", True)
    for (oa, sca), (ob, scb) in zip(outs_a, outs_b):
        assert_close(oa[:, 0].float().cpu().numpy(), ea, what="stream a output")
        assert_close(sca.cpu().numpy(), esa, what="stream a scores")
        assert_close(ob[:, 0].float().cpu().numpy(), eb, what="stream b output")
        assert_close(scb.cpu().numpy(), esb, what="stream b scores")
    assert workspace_error_word(device) == 0


# -- shapes, formats and modes ------------------------------------------------

@pytest.mark.parametrize("groups", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("fmt", ["absmax_i8", "ref_u8"])
def test_gqa_dims_formats(device, groups, head_dim, fmt):
    kv = 2
    nb = 37
    gen = torch.Generator().manual_seed(groups * 1000 + head_dim)
    lengths = torch.randint(1, 17, (3, nb), generator=gen)
    lengths[:, :-1] = torch.where(torch.rand((3, nb - 1), generator=gen) < 0.8, 16, lengths[:, :-1])
    case = W.make_tiered_case(f"gqa{groups}_d{head_dim}", 3, kv * groups, kv, head_dim, nb, 9, 17,
                              seed=groups + head_dim, lengths=lengths, max_blocks=nb + 5)
    for cold in ("masked", "zero_logit"):
        _check(case, fmt, device, cold_mode=cold, return_scores=True)
    # The same case split over two workgroups per unit (partials merged by the
    # last arrival, score sums finalised from the staged block statistics).
    _check(case, fmt, device, cold_mode="zero_logit", return_scores=True, splits=2)


@pytest.mark.parametrize("splits", [1, 2, 3, 7])
def test_split_invariance(device, splits):
    case = W.make_tiered_case("splits", 2, 32, 8, 128, 100, 12, 60, seed=7)
    out_auto = _check(case, "absmax_i8", device)[0]
    out_s = _check(case, "absmax_i8", device, splits=splits)[0]
    # Both match the oracle above.  Between themselves they differ by fp32
    # re-association, the fp16 rounding of the output, and the fp16 rounding
    # of the probabilities the PV product uses, which are taken relative to
    # each wave's running maximum and so depend on how tiles are partitioned
    # (splits, dynamic hand-out, work sharing): 2^-11 relative per
    # probability, about 2^-11 * max|V| (~4) in the worst case per output.
    assert_close(out_s.float().cpu().numpy(), out_auto.float().cpu().numpy(), atol=5e-4, rtol=2.0 ** -9,
                 what="split vs auto")


@pytest.mark.parametrize("cold", ["masked", "zero_logit"])
def test_scores_many_splits(device, cold):
    # More splits than a wave has lanes: the merge's per-head (M, L) reduction
    # takes its strided path, and the score finalisation batches its loads
    # over many blocks per thread.
    lengths = torch.full((2, 300), 16, dtype=torch.int32)
    lengths[:, 7::13] = 5
    case = W.make_tiered_case("many_splits", 2, 8, 2, 64, 300, 40, 150, seed=41, lengths=lengths,
                              max_blocks=310)
    _check(case, "absmax_i8", device, cold_mode=cold, return_scores=True, splits=70)


@pytest.mark.parametrize("groups", [4, 16])
def test_long_row_list_build(device, groups):
    # A table row longer than the list build's preloaded chunks (4 x 512
    # entries with 8 waves, 4 x 256 with 4 waves at group 16): the build
    # loops, and ranks continue across its iterations.
    case = W.make_tiered_case(f"long_row_g{groups}", 1, groups, 1, 64, 2600, 100, 900, seed=43 + groups,
                              recent_hot=4)
    _check(case, "absmax_i8", device, return_scores=True)
    _check(case, "ref_u8", device, cold_mode="zero_logit", return_scores=True)


@pytest.mark.parametrize("scores", [False, True])
def test_one_pass_long_rows_split_ranges(device, scores):
    # Rows longer than one 512-entry chunk but within one pass of the long-row
    # build (at most 4 x 512 blocks): each split owns a contiguous range of
    # the HOT ranks and of the WARM ranks.  Many split counts, ragged lengths
    # (zero-length blocks are skipped), and a sparse row where most splits own
    # nothing.
    g = torch.Generator().manual_seed(5)
    lengths = torch.randint(0, 17, (2, 1500), generator=g, dtype=torch.int32)
    lengths[:, -1] = 3
    dense = W.make_tiered_case("one_pass", 2, 8, 2, 64, 1500, 60, 500, seed=81, lengths=lengths, max_blocks=1510)
    sparse = W.make_tiered_case("one_pass_sparse", 1, 8, 2, 64, 700, 2, 3, seed=82, recent_hot=1)
    for case, fmt, cold in ((dense, "absmax_i8", "masked"), (sparse, "ref_u8", "zero_logit")):
        warm = oracle_warm(case, fmt)
        args = to_gpu_inputs(case, warm, device)
        res = oracle_decode(case, warm, fmt, cold, scores)
        exp_out, exp_sc = res if scores else (res, None)
        for splits in (1, 2, 3, 5, 8, 13):
            print(f"[decode] one-pass long rows: case={case.name} fmt={fmt} splits={splits} scores={scores}",
                  flush=True)
            out, sc = tierkv_decode_attention(**args, return_scores=scores, cold_mode=cold, splits=splits)
            torch.cuda.synchronize()
            assert_close(out[:, 0].float().cpu().numpy(), exp_out, what=f"{case.name} splits={splits} output")
            if scores:
                sc = sc.cpu().numpy()
                assert_close(sc[None] if sc.ndim == 2 else sc, exp_sc, what=f"{case.name} splits={splits} score_sums")
            assert workspace_error_word(device) == 0


def test_repeated_calls_reuse_bound_arguments(device):
    # A decode loop passes the same tables and pools every step with a new
    # query and block count: the second and later calls skip the tensors'
    # validation (tierkv_hip's rebind entries) and must give what a full
    # bind gives; per-call arguments are still checked, and a replaced pool
    # tensor is bound anew.
    import paged_tierkv_amd.tierkv_hip as th
    case = W.make_tiered_case("rebind", 1, 8, 2, 64, 40, 8, 20, seed=91, recent_hot=2)
    warm = oracle_warm(case, "absmax_i8")
    args = to_gpu_inputs(case, warm, device)
    th._REBIND.clear()
    first, _ = tierkv_decode_attention(**args, cold_mode="masked")
    assert len(th._REBIND) == 1
    for nb in (40, 25, 40):
        a = dict(args, num_blocks=nb, query_states=args["query_states"].clone())
        got, _ = tierkv_decode_attention(**a, cold_mode="masked")
        case_nb = W.make_tiered_case("rebind", 1, 8, 2, 64, 40, 8, 20, seed=91, recent_hot=2)
        case_nb.num_blocks = nb
        exp = oracle_decode(case_nb, warm, "absmax_i8", "masked")
        assert_close(got[:, 0].float().cpu().numpy(), exp, what=f"rebind num_blocks={nb}")
    assert len(th._REBIND) == 1
    with pytest.raises(ValueError, match="exceeds"):
        tierkv_decode_attention(**dict(args, num_blocks=41), cold_mode="masked")
    with pytest.raises(ValueError, match="positive"):
        tierkv_decode_attention(**dict(args, num_blocks=0), cold_mode="masked")
    moved = dict(args, hot_k_pool=args["hot_k_pool"].clone())
    again, _ = tierkv_decode_attention(**moved, cold_mode="masked")
    assert len(th._REBIND) == 2
    torch.cuda.synchronize()
    assert torch.allclose(again.float(), first.float(), atol=2e-3, rtol=1e-2)


@pytest.mark.parametrize("fmt", ["absmax_i8", "ref_u8"])
def test_large_warm_v_scales(device, fmt):
    # WARM V blocks whose scale exceeds 2 take the kernel's unfolded path
    # (the scale applied to V before the MFMA, so fp16 P cannot overflow);
    # every other slot's V stays small, so the waves meet both paths, and
    # the offset sums of the folded tiles must not absorb the unfolded ones.
    case = W.make_tiered_case("big_v", 2, 8, 2, 64, 48, 6, 30, seed=95, recent_hot=2)
    v = case.warm_src_v.float()
    v[0::2] *= 600.0
    case.warm_src_v = v.to(torch.float16)
    warm = oracle_warm(case, fmt)
    sv = np.asarray(warm[4], dtype=np.float32)
    assert (sv > 2).any() and (sv <= 2).any()
    # The unfolded path rounds each dequantized V value to fp16 before the
    # MFMA (the oracle keeps it in fp32): an output element can differ by up
    # to half an fp16 ulp of the largest |V|, 2^-11 * max|V|.  A wrong scale,
    # offset or tile would be off by far more.
    vmax = float(np.abs(case.warm_src_v.float().numpy()).max())
    atol = 2.0 ** -11 * vmax
    cold = "zero_logit" if fmt == "ref_u8" else "masked"
    args = to_gpu_inputs(case, warm, device)
    exp_out, exp_sc = oracle_decode(case, warm, fmt, cold, True)
    for splits in (None, 3):
        print(f"[decode] large WARM V scales fmt={fmt} splits={splits} atol={atol:.3f}", flush=True)
        out, sc = tierkv_decode_attention(**args, return_scores=True, cold_mode=cold, splits=splits)
        torch.cuda.synchronize()
        report(f"big_v {fmt} splits={splits} output",
               assert_close(out[:, 0].float().cpu().numpy(), exp_out, atol=atol, what="big_v output"))
        report(f"big_v {fmt} splits={splits} score_sums",
               assert_close(sc.cpu().numpy(), exp_sc, what="big_v score_sums"))
        assert workspace_error_word(device) == 0


@pytest.mark.parametrize("fmt", ["absmax_i8", "ref_u8"])
def test_split_list_capacity(device, fmt):
    # 1 HOT + 1023 WARM blocks asked to run in 2 splits: split 0 would get
    # ceil(1/2) + ceil(1023/2) = 513 list entries, one more than the LDS list
    # holds; the plan raises the split count so that HOT (front) and WARM
    # (back) entries never meet.
    case = W.make_tiered_case("list_cap", 1, 4, 1, 64, 1024, 1, 1023, seed=71)
    _check(case, fmt, device, cold_mode="zero_logit", return_scores=True, splits=2)


def test_split_launch_in_sequence_chunks(device):
    # More (sequence, kv head) units than the split-arrival counter region
    # holds (65536): the host launches the batch in chunks of whole
    # sequences on offset pointers.  Every sequence shares one table row and
    # the pools, with its own scaled query; sequences on both sides of the
    # chunk boundary are checked against the oracle.
    one = W.make_tiered_case("chunks", 1, 2, 1, 64, 40, 10, 20, seed=51, max_blocks=44)
    warm = oracle_warm(one, "absmax_i8")
    B = 65536 + 5
    scale = 1.0 + 0.05 * (torch.arange(B) % 13).to(torch.float16)
    args = to_gpu_inputs(one, warm, device)
    args["query_states"] = (args["query_states"] * scale.to(device).view(B, 1, 1, 1)).contiguous()
    for k in ("block_table", "block_states", "block_lengths"):
        args[k] = args[k].expand(B, -1).contiguous()
    out, sc = tierkv_decode_attention(**args, return_scores=True, cold_mode="masked", splits=2)
    torch.cuda.synchronize()
    assert workspace_error_word(device) == 0
    for b in (0, 1, 65534, 65535, 65536, 65537, B - 1):
        sub = W.make_tiered_case("chunks", 1, 2, 1, 64, 40, 10, 20, seed=51, max_blocks=44)
        sub.query = (sub.query * scale[b]).to(torch.float16)
        exp_out, exp_sc = oracle_decode(sub, warm, "absmax_i8", "masked", True)
        assert_close(out[b, 0].float().cpu().numpy(), exp_out[0], what=f"seq {b} out")
        assert_close(sc[b].cpu().numpy(), exp_sc[0], what=f"seq {b} scores")


def test_seq_num_blocks_ragged(device):
    case = W.make_tiered_case("ragged", 4, 16, 4, 64, 48, 8, 24, seed=11)
    snb = [48, 1, 17, 30]
    warm = oracle_warm(case, "absmax_i8")
    args = to_gpu_inputs(case, warm, device)
    out, sc = tierkv_decode_attention(**args, return_scores=True, cold_mode="masked", seq_num_blocks=snb)
    torch.cuda.synchronize()
    for b, n in enumerate(snb):
        sub = W.make_tiered_case("ragged", 4, 16, 4, 64, 48, 8, 24, seed=11)
        sub.num_blocks = n
        exp_out, exp_sc = oracle_decode(sub, warm, "absmax_i8", "masked", True, seqs=[b])
        assert_close(out[b, 0].float().cpu().numpy(), exp_out[0], what=f"seq {b} out")
        assert_close(sc[b].cpu().numpy(), exp_sc[0], what=f"seq {b} scores")
        assert float(sc[b, :, n:].abs().sum()) == 0.0


def test_all_cold(device):
    case = W.make_tiered_case("allcold", 2, 8, 4, 64, 6, 0, 0, seed=3)
    case.block_states[:, :6] = W.COLD
    for cold in ("masked", "zero_logit"):
        _, out, sc = _run(case, "absmax_i8", device, cold_mode=cold, return_scores=True)
        assert float(out.float().abs().max()) == 0.0
        if cold == "zero_logit":
            s = sc.cpu().numpy()[:, :, :6].sum(-1)
            np.testing.assert_allclose(s, 1.0, atol=1e-5)


def test_growable_workspace_grows_on_a_side_stream(device):
    """A growable workspace bound to launches on a side stream grows there:
    before its old buffer is dropped it is recorded on every stream that used
    it, so the caching allocator hands it out again only after their queued
    launches; every launch matches the oracle."""
    from paged_tierkv_amd.tierkv_hip import DecodeWorkspace

    small = W.make_tiered_case("ws_small", 2, 16, 4, 64, 30, 6, 14, seed=81)
    big = W.make_tiered_case("ws_big", 4, 32, 8, 128, 600, 60, 300, seed=82)
    runs = [(small, "absmax_i8", "masked", 2), (big, "ref_u8", "zero_logit", 6), (small, "ref_u8", "masked", 1)]
    prepared = []
    for case, fmt, cold, splits in runs:
        warm = oracle_warm(case, fmt)
        prepared.append((case, warm, fmt, cold, splits, to_gpu_inputs(case, warm, device)))
    torch.cuda.synchronize()
    ws = DecodeWorkspace(device)            # 256 bytes: the launches below grow it
    side = torch.cuda.Stream(device)
    outs = []
    with torch.cuda.stream(side):
        for case, warm, fmt, cold, splits, inputs in prepared:
            print(f"[ws-side] case={case.name} fmt={fmt} cold={cold} splits={splits} bytes={ws.nbytes}", flush=True)
            outs.append(tierkv_decode_attention(**inputs, return_scores=True, cold_mode=cold, splits=splits,
                                                workspace=ws))
    assert ws.growable and ws.nbytes > 256 and any(s == side for s in ws._streams)
    side.synchronize()
    assert ws.error_word() == 0
    for (case, warm, fmt, cold, splits, _), (out, sc) in zip(prepared, outs):
        exp_out, exp_sc = oracle_decode(case, warm, fmt, cold, True)
        assert_close(out[:, 0].float().cpu().numpy(), exp_out, what=f"{case.name} side-stream output")
        assert_close(sc.cpu().numpy(), exp_sc, what=f"{case.name} side-stream score_sums")


def test_invalid_slot_is_skipped_and_flagged(device, monkeypatch):
    case = W.make_tiered_case("badslot", 1, 8, 4, 64, 4, 4, 0, seed=5)
    case.block_table[0, 2] = 10_000   # out of range HOT slot: never dereferenced
    warm = oracle_warm(case, "absmax_i8")
    args = to_gpu_inputs(case, warm, device)
    monkeypatch.setenv("TIERKV_CHECK_ERRORS", "1")
    with pytest.raises(RuntimeError, match="out-of-range"):
        tierkv_decode_attention(**args, cold_mode="masked")


# -- the reference's own decode tests (main.py:452-634; tierkv_triton.py:823-1097)

def _ref_geometry_case(states, lengths, kv_heads, q_heads, head_dim, seed):
    nb = len(states)
    case = W.make_tiered_case("refgeom", 1, q_heads, kv_heads, head_dim, nb, nb, 0, seed=seed,
                              lengths=[lengths], max_blocks=nb + 4, layout="dense",
                              dense_pool_blocks=nb + 4)
    case.block_states[0, :nb] = torch.tensor(states, dtype=torch.int32)
    return case


@pytest.mark.parametrize("states,lengths", [
    ([0, 0], [16, 5]),                       # 21 tokens all HOT (main.py:498-535)
    ([1, 1], [16, 5]),                       # all WARM (main.py:545-566)
    ([0, 1, 2], [16, 16, 9]),                # mixed H/W/C (main.py:568-598)
    ([0, 1, 0, 1, 0, 0], [16] * 5 + [1]),   # > 4 blocks (main.py:600-624)
])
def test_reference_main_geometry(device, states, lengths):
    # kv_heads 2, q heads 4, head_dim 16: generic kernel path.
    case = _ref_geometry_case(states, lengths, 2, 4, 16, seed=len(states))
    _check(case, "ref_u8", device, cold_mode="zero_logit", return_scores=True)


@pytest.mark.parametrize("states", [
    [0] * 6,                                 # 2.1 all-HOT with scores (tierkv_triton.py:901-938)
    [0, 1, 2, 0, 1],                         # 2.2 HOT/WARM/COLD/HOT/WARM (943-989)
    [0, 1, 0, 0, 1, 0, 0, 1],                # 2.3 split path, 8 blocks (994-1050)
])
def test_reference_preservation_geometry(device, states):
    # kv_heads 4, q heads 8, head_dim 64, block 16: fast path.
    case = _ref_geometry_case(states, [16] * len(states), 4, 8, 64, seed=10 + len(states))
    _check(case, "ref_u8", device, cold_mode="zero_logit", return_scores=True)
    # The reference API: 1-D tables, scores [H, max_blocks], (out, None) without scores.
    args = to_gpu_inputs(case, oracle_warm(case, "ref_u8"), device)
    for k in ("block_table", "block_states", "block_lengths"):
        args[k] = args[k][0].contiguous()
    out, sc = tierkv_decode_attention(**args, return_scores=True)
    assert sc.shape == (8, len(states) + 4)
    np.testing.assert_allclose(sc[:, : len(states)].sum(-1).cpu().numpy(), 1.0, atol=2e-2)
    exp_out, exp_sc = oracle_decode(case, oracle_warm(case, "ref_u8"), "ref_u8", "zero_logit", True)
    assert_close(out[:, 0].float().cpu().numpy(), exp_out, what="1-D table output")
    assert_close(sc.cpu().numpy()[None], exp_sc, what="1-D table scores")
    out2, none = tierkv_decode_attention(**args, return_scores=False)
    assert none is None and out2.shape == (1, 1, 8, 64)


# -- workspace reuse ------------------------------------------------------------

def test_workspace_reuse_across_shapes(device):
    # The per-device workspace is shared by launches of every shape; split
    # launches (several workgroups per unit, arrival counters that each
    # launch's last arrivals reset) and score launches are interleaved with
    # single-split ones: no launch may depend on what another layout left in
    # the workspace.
    big = W.make_tiered_case("reuse_big", 16, 32, 8, 128, 64, 6, 40, seed=31)
    small = W.make_tiered_case("reuse_small", 3, 16, 4, 128, 48, 4, 30, seed=32)
    split = W.make_tiered_case("reuse_split", 2, 32, 8, 128, 100, 12, 60, seed=33)
    for case, kw in ((big, {}), (small, {}), (split, {}), (big, {"return_scores": True}),
                     (split, {"return_scores": True}), (small, {"return_scores": True}),
                     (split, {"splits": 3}), (big, {}), (split, {})):
        _check(case, "absmax_i8", device, seqs=[0, case.batch - 1], **kw)

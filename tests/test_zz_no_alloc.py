"""The allocation-free decode entry point, tierkv_decode_attention_noalloc,
against tierkv_decode_attention: both called through the C ABI on the same
bound inputs, two or more calls in a row on the library's one scratch array
(the later ones smaller), each also checked against the CPU oracle.

Also: the scratch array's error word (tierkv_decode_noalloc_error_word),
and the first call on a device in a fresh process, which zeroes the array
before any launch on another stream can use it.

Bar: per-block score sums bit-exact (their reduction order is fixed);
outputs within the split-invariance bound of each other (each wave's
running maximum depends on the dynamic tile hand-out) and within 2e-3
absolute / 1e-2 relative of the oracle."""

from __future__ import annotations

import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from paged_tierkv_amd import _lib
from paged_tierkv_amd import workloads as W
from paged_tierkv_amd.tierkv_hip import (NOALLOC, DecodeWorkspace, PreparedDecode, _bind, noalloc_error_word,
                                         tierkv_decode_attention, workspace_error_word)

from helpers import assert_close, oracle_decode, oracle_warm, report, to_gpu_inputs

pytestmark = pytest.mark.gpu

SCRATCH_LIMIT = 16 << 20


def _pair(case, fmt, device, cold, scores, splits):
    """One launch through each entry point; returns both (out, score_sums)."""
    warm = oracle_warm(case, fmt)
    inputs = to_gpu_inputs(case, warm, device)
    kw = dict(return_scores=scores, cold_mode=cold, splits=splits)
    lib = _lib.lib()
    need = lib.tierkv_decode_workspace_bytes(case.batch, case.query.shape[1], case.hot_k.shape[1], case.num_blocks,
                                             case.hot_k.shape[2], case.hot_k.shape[3], int(scores), splits or 0)
    assert 0 < need <= SCRATCH_LIMIT
    ws = DecodeWorkspace(device, need, growable=False)
    args_w, out_w, sc_w, _, _, keep_w = _bind(**inputs, workspace=ws, **kw)
    args_n, out_n, sc_n, ws_n, _, keep_n = _bind(**inputs, workspace=NOALLOC, **kw)
    assert ws_n is None and len(args_n) == len(args_w) - 2
    stream = _lib.stream_of(device)
    print(f"[noalloc] case={case.name} fmt={fmt} cold={cold} scores={scores} splits={splits} need={need}",
          flush=True)
    _lib.check(lib.tierkv_decode_attention(*args_w, stream), "tierkv_decode_attention")
    _lib.check(lib.tierkv_decode_attention_noalloc(*args_n, stream), "tierkv_decode_attention_noalloc")
    torch.cuda.synchronize()
    assert ws.error_word() == 0
    got_n = out_n[:, 0].float().cpu().numpy()
    got_w = out_w[:, 0].float().cpu().numpy()
    assert_close(got_n, got_w, atol=5e-4, rtol=2.0 ** -9, what=f"{case.name} noalloc vs workspace")
    res = oracle_decode(case, warm, fmt, cold, scores)
    exp = res[0] if scores else res
    report(f"{case.name} noalloc output", assert_close(got_n, exp, what=f"{case.name} noalloc output"))
    if scores:
        a, b = sc_n.cpu().numpy(), sc_w.cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{case.name}: score sums differ"
        report(f"{case.name} noalloc score_sums", assert_close(a, res[1], what=f"{case.name} score_sums"))
    del keep_w, keep_n


def _cases():
    split = W.make_tiered_case("noalloc_split", 4, 32, 8, 128, 256, 24, 160, seed=91, recent_hot=4)
    lengths = torch.full((3, 40), 16, dtype=torch.int32)
    lengths[:, 5::7] = 3
    small = W.make_tiered_case("noalloc_small", 3, 16, 4, 64, 40, 8, 20, seed=92, lengths=lengths, max_blocks=44)
    return split, small


def test_noalloc_matches_workspace_entry_point(device):
    split, small = _cases()
    # The larger launch first (several splits: arrival counters and staged
    # score partials in the scratch), then smaller ones that reuse what it
    # left there, then the large one again without scores.
    _pair(split, "absmax_i8", device, "masked", True, 3)
    _pair(small, "absmax_i8", device, "masked", True, None)
    _pair(small, "ref_u8", device, "zero_logit", True, 2)
    _pair(split, "ref_u8", device, "zero_logit", False, None)


def test_noalloc_python_routes(device):
    # workspace=NOALLOC through the public wrapper and a prepared launch.
    _, small = _cases()
    warm = oracle_warm(small, "absmax_i8")
    inputs = to_gpu_inputs(small, warm, device)
    out_d, sc_d = tierkv_decode_attention(**inputs, return_scores=True, cold_mode="masked")
    out_n, sc_n = tierkv_decode_attention(**inputs, return_scores=True, cold_mode="masked", workspace=NOALLOC)
    plan = PreparedDecode(**inputs, return_scores=True, cold_mode="masked", workspace=NOALLOC)
    assert plan.workspace is None
    out_p, sc_p = plan.launch()
    torch.cuda.synchronize()
    for o, s in ((out_n, sc_n), (out_p, sc_p)):
        assert torch.equal(s, sc_d)
        assert_close(o.float().cpu().numpy(), out_d.float().cpu().numpy(), atol=5e-4, rtol=2.0 ** -9,
                     what="noalloc route")


def test_noalloc_rejects_oversize(device):
    # Eight 8192-block sequences with scores need more than the 16 MiB the
    # entry point holds: refused before any launch.  Every block is COLD, so
    # the inputs are valid however the launch were treated.
    batch, heads, kv_heads, nb, bs, d = 8, 32, 8, 8192, 16, 128
    lib = _lib.lib()
    assert lib.tierkv_decode_workspace_bytes(batch, heads, kv_heads, nb, bs, d, 1, 0) > SCRATCH_LIMIT
    table = torch.full((batch, nb), -1, dtype=torch.int32, device=device)
    states = torch.full((batch, nb), 2, dtype=torch.int32, device=device)
    lengths = torch.full((batch, nb), bs, dtype=torch.int32, device=device)
    hot = torch.zeros((1, kv_heads, bs, d), dtype=torch.float16, device=device)
    warm = torch.zeros((1, kv_heads, bs, d), dtype=torch.int8, device=device)
    scale = torch.ones((1, kv_heads), dtype=torch.float32, device=device)
    query = torch.randn((batch, heads, 1, d), device=device).half()
    with pytest.raises(RuntimeError, match="allocation-free entry point holds"):
        tierkv_decode_attention(query, table, states, lengths, hot, hot, warm, warm, scale, None, scale, None,
                                nb, heads // kv_heads, d ** -0.5, True, cold_mode="masked", workspace=NOALLOC)
    # The same launch without scores fits.
    need = lib.tierkv_decode_workspace_bytes(batch, heads, kv_heads, nb, bs, d, 0, 0)
    if need <= SCRATCH_LIMIT:
        out, _ = tierkv_decode_attention(query, table, states, lengths, hot, hot, warm, warm, scale, None, scale,
                                         None, nb, heads // kv_heads, d ** -0.5, False, cold_mode="masked",
                                         workspace=NOALLOC)
        torch.cuda.synchronize()
        assert out.shape == (batch, 1, heads, d)


def test_noalloc_error_word(device, monkeypatch):
    """A block whose slot is out of range is skipped by an allocation-free
    launch and flagged in the scratch array's error word, which
    tierkv_decode_noalloc_error_word reads and clears."""
    case = W.make_tiered_case("noalloc_badslot", 1, 8, 4, 64, 4, 4, 0, seed=5)
    case.block_table[0, 2] = 10_000   # out-of-range HOT slot: never dereferenced
    args = to_gpu_inputs(case, oracle_warm(case, "absmax_i8"), device)
    print("[noalloc] bad slot, error word", flush=True)
    assert noalloc_error_word(device) == 0
    tierkv_decode_attention(**args, cold_mode="masked", workspace=NOALLOC)
    assert noalloc_error_word(device, clear=False) == 1
    assert workspace_error_word(device) == 1      # read and cleared with the workspaces' words
    assert noalloc_error_word(device) == 0
    monkeypatch.setenv("TIERKV_CHECK_ERRORS", "1")
    with pytest.raises(RuntimeError, match="out-of-range"):
        tierkv_decode_attention(**args, cold_mode="masked", workspace=NOALLOC)
    assert noalloc_error_word(device) == 0


_FIRST_CALL_SCRIPT = r"""
import torch
from paged_tierkv_amd import workloads as W
from paged_tierkv_amd.tierkv_hip import NOALLOC, tierkv_decode_attention, workspace_error_word
from helpers import assert_close, oracle_decode, oracle_warm, to_gpu_inputs

dev = torch.device("cuda:0")
a = W.make_tiered_case("first_a", 1, 16, 4, 64, 20, 6, 10, seed=95)          # unsplit, no scores
b = W.make_tiered_case("first_b", 4, 32, 8, 128, 512, 60, 300, seed=96)      # split, with scores
wa, wb = oracle_warm(a, "absmax_i8"), oracle_warm(b, "ref_u8")
ia, ib = to_gpu_inputs(a, wa, dev), to_gpu_inputs(b, wb, dev)
torch.cuda.synchronize()
sa, sb = torch.cuda.Stream(dev), torch.cuda.Stream(dev)
print("first noalloc call on stream A, then at once a split launch on stream B", flush=True)
with torch.cuda.stream(sa):
    out_a, _ = tierkv_decode_attention(**ia, cold_mode="masked", splits=1, workspace=NOALLOC)
with torch.cuda.stream(sb):
    out_b, sc_b = tierkv_decode_attention(**ib, return_scores=True, cold_mode="zero_logit", splits=4,
                                          workspace=NOALLOC)
torch.cuda.synchronize()
assert workspace_error_word(dev) == 0
assert_close(out_a[:, 0].float().cpu().numpy(), oracle_decode(a, wa, "absmax_i8", "masked"), what="stream A")
exp_out, exp_sc = oracle_decode(b, wb, "ref_u8", "zero_logit", True)
assert_close(out_b[:, 0].float().cpu().numpy(), exp_out, what="stream B output")
assert_close(sc_b.cpu().numpy(), exp_sc, what="stream B score_sums")
print("FIRST-CALL OK", flush=True)
"""


def test_noalloc_first_call_then_other_stream(device):
    """In a fresh process (the scratch array not yet zeroed): the first
    allocation-free call, on stream A, zeroes the array and waits for it
    before publishing its address, so a split launch issued right after on
    stream B -- ordered on the host only -- finds its arrival counters zero.
    (The first launch is unsplit and without scores: it shares nothing with
    the second but the error word, so the two may overlap.)"""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([root, os.path.join(root, "tests"),
                                                       os.environ.get("PYTHONPATH", "")]))
    print("[noalloc] fresh process: first call on stream A, split launch on stream B", flush=True)
    proc = subprocess.run([sys.executable, "-c", _FIRST_CALL_SCRIPT], cwd=root, env=env, capture_output=True,
                          text=True, timeout=300)
    print(proc.stdout[-2000:], proc.stderr[-2000:], flush=True)
    assert proc.returncode == 0 and "FIRST-CALL OK" in proc.stdout


def test_noalloc_deterministic_matches_workspace_bits(device):
    """With the deterministic tile hand-out both entry points compute the
    same sums in the same order: their outputs are the same bits, on two
    calls in a row (the second smaller)."""
    split, small = _cases()
    for case, fmt, cold in ((split, "absmax_i8", "masked"), (small, "ref_u8", "zero_logit")):
        print(f"[noalloc] deterministic {case.name} {fmt}", flush=True)
        warm = oracle_warm(case, fmt)
        inputs = to_gpu_inputs(case, warm, device)
        out_w, sc_w = tierkv_decode_attention(**inputs, return_scores=True, cold_mode=cold, deterministic=True)
        out_n, sc_n = tierkv_decode_attention(**inputs, return_scores=True, cold_mode=cold, deterministic=True,
                                              workspace=NOALLOC)
        torch.cuda.synchronize()
        assert torch.equal(out_w.view(torch.int16), out_n.view(torch.int16))
        assert torch.equal(sc_w.view(torch.int32), sc_n.view(torch.int32))

"""Decode-workspace ownership rules, checked on the CPU (no kernel launches).

* A fixed workspace never replaces its buffer: a launch that needs more
  raises, so a captured graph can never replay on a released buffer.
* A growable workspace carries its error flags into the new buffer.
* A workspace first bound under stream capture becomes fixed, so a later,
  larger eager launch cannot free memory a captured graph replays on.
* The batched runtime sizes its fixed workspace once, for ``max_blocks``
  with score sums; every smaller launch of the same geometry (any block
  count, with or without scores) fits in it, so nothing it launches can ask
  for more.
"""

from __future__ import annotations

import pytest
import torch

from paged_tierkv_amd.tierkv_hip import DecodeWorkspace


def test_fixed_workspace_never_replaces_its_buffer():
    ws = DecodeWorkspace("cpu", 4096, growable=False)
    before = ws.data_ptr()
    ws.reserve(4096)
    ws.reserve(100)
    assert ws.data_ptr() == before
    with pytest.raises(RuntimeError, match="fixed workspace"):
        ws.reserve(4097)
    assert ws.data_ptr() == before and ws.nbytes == 4096


def test_growable_workspace_keeps_error_flags():
    ws = DecodeWorkspace("cpu", 256)
    ws.buf[:4].view(torch.int32).fill_(2)
    ws.reserve(1 << 16)
    assert ws.nbytes == 1 << 16
    assert int(ws.buf[:4].view(torch.int32).item()) == 2
    assert int(ws.buf[4:].abs().sum()) == 0
    assert ws.error_word() == 2
    assert ws.error_word() == 0


def test_capture_pins_a_growable_workspace(monkeypatch):
    ws = DecodeWorkspace("cpu", 4096)
    assert ws.growable
    monkeypatch.setattr(DecodeWorkspace, "_capturing", lambda self: True)
    ws.reserve(1024)                    # bound under capture: fits, and is fixed from now on
    assert not ws.growable
    with pytest.raises(RuntimeError, match="during HIP graph capture"):
        ws.reserve(8192)
    monkeypatch.setattr(DecodeWorkspace, "_capturing", lambda self: False)
    before = ws.data_ptr()
    with pytest.raises(RuntimeError, match="fixed workspace"):
        ws.reserve(8192)                # eager growth after the capture is refused
    assert ws.data_ptr() == before and ws.nbytes == 4096


@pytest.mark.parametrize("batch,heads,kv,dim,max_blocks", [
    (16, 32, 8, 128, 144),     # C5: Llama-3-8B, 2048 + 256 tokens
    (1, 32, 4, 64, 33),        # TinyLlama shape, batch 1
    (4, 32, 8, 128, 2048),     # C4 rows
    (3, 48, 3, 128, 700),      # GQA 16, four waves per workgroup
])
def test_runtime_workspace_covers_every_launch(batch, heads, kv, dim, max_blocks):
    full = DecodeWorkspace.bytes_for(batch, heads, kv, max_blocks, dim, return_scores=True)
    for nb in range(1, max_blocks + 1):
        for scores in (False, True):
            assert DecodeWorkspace.bytes_for(batch, heads, kv, nb, dim, return_scores=scores) <= full, (nb, scores)


def test_graph_runner_reserves_before_capture(monkeypatch):
    """DecodeGraphRunner reserves the runtime's decode workspace in its
    constructor, before any step could be captured."""
    from paged_tierkv_amd import hf_llama

    calls = []

    class Rt:
        is_batched = True
        batch = 2
        device = torch.device("cpu")
        fixed_launch_bound = False

        def reserve_decode_workspace(self, heads):
            calls.append(heads)

    class Cfg:
        num_attention_heads = 32

    class Model:
        config = Cfg()

    runner = hf_llama.DecodeGraphRunner(Model(), Rt())
    assert calls == [32]
    assert runner.rt.fixed_launch_bound

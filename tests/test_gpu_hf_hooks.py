"""GPU end-to-end checks of the HF hooks (paged_tierkv_amd.hf_llama) in a
small random-init Llama (fp16, GQA group 4, head_dim 64), teacher-forced so
every run sees the same token sequence:

* reference-API runtime, HOT only: logits match the stock HF model with its
  DynamicCache (fp16 model arithmetic; the decode kernel accumulates in fp32);
* reference-API runtime with HOT+WARM tiering: the kernel backend matches
  the reference's eager backend (reconstructed K/V + the model's attention)
  on the same tier layout, and WARM blocks really are in use;
* batched runtime, everything HOT: logits match stock HF batched decoding;
* batched runtime with HOT/WARM/COLD tiering and device policy ticks: runs
  without allocator errors, keeps logits finite and compresses the cache."""

from __future__ import annotations

import pytest
import torch

transformers = pytest.importorskip("transformers")

from paged_tierkv_amd import hf_llama, tierkv_policy as tp  # noqa: E402
from paged_tierkv_amd.block_manager import BlockManager  # noqa: E402
from paged_tierkv_amd.runtime import BatchedTieredKVRuntime  # noqa: E402

pytestmark = pytest.mark.gpu

PROMPT, STEPS = 100, 24


@pytest.fixture(scope="module")
def model(device):
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(hidden_size=512, intermediate_size=1024, num_hidden_layers=2, num_attention_heads=8,
                      num_key_value_heads=2, head_dim=64, vocab_size=1000, max_position_embeddings=1024)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    m = LlamaForCausalLM(cfg).to(device=device, dtype=torch.float16).eval()
    hf_llama.install()
    yield m
    hf_llama.uninstall()
    tp.reset_global_tierkv()


def _tokens(batch, device):
    g = torch.Generator().manual_seed(11)
    return torch.randint(0, 1000, (batch, PROMPT + STEPS), generator=g).to(device)


def _teacher_forced(model, ids, cache):
    """Prefill ids[:, :PROMPT], then feed ids[:, PROMPT + s] one at a time;
    returns the last-position logits of every forward [STEPS + 1, B, V]."""
    outs = []
    with torch.no_grad():
        out = model(input_ids=ids[:, :PROMPT], past_key_values=cache, use_cache=True, logits_to_keep=1)
        outs.append(out.logits[:, -1].float())
        cache = out.past_key_values
        for s in range(STEPS):
            out = model(input_ids=ids[:, PROMPT + s: PROMPT + s + 1], past_key_values=cache, use_cache=True,
                        logits_to_keep=1)
            outs.append(out.logits[:, -1].float())
            cache = out.past_key_values
    return torch.stack(outs)


def _dropin_runtime(model, **kw):
    cfg = model.config
    return tp.TieredKVRuntime(block_manager=BlockManager(total_blocks=4096), num_layers=cfg.num_hidden_layers,
                              block_size=16, max_seq_len=PROMPT + STEPS + 16, **kw)


def test_dropin_hot_only_matches_stock(model, device):
    print("[hf] drop-in hot_only vs stock", flush=True)
    from transformers import DynamicCache

    ids = _tokens(1, device)
    ref = _teacher_forced(model, ids, DynamicCache(config=model.config))
    rt = _dropin_runtime(model, hot_budget=3, attention_backend="triton", policy_interval=8, policy_mode="hot_only")
    got = _teacher_forced(model, ids, rt.cache)
    torch.testing.assert_close(got, ref, atol=2e-2, rtol=2e-2)
    assert rt.cache.get_seq_length() == PROMPT + STEPS


def test_dropin_tiered_kernel_matches_eager_backend(model, device):
    print("[hf] drop-in hot_warm kernel vs eager", flush=True)
    ids = _tokens(1, device)
    kw = dict(hot_budget=3, policy_interval=10_000, policy_mode="hot_warm")
    rt_k = _dropin_runtime(model, attention_backend="triton", **kw)
    got = _teacher_forced(model, ids, rt_k.cache)
    rt_e = _dropin_runtime(model, attention_backend="eager", **kw)
    ref = _teacher_forced(model, ids, rt_e.cache)
    torch.testing.assert_close(got, ref, atol=2e-2, rtol=2e-2)
    m = rt_k.collect_memory_metrics()
    assert m["warm_blocks"] > 0 and m["logical_compression_x"] > 1.0


@pytest.mark.parametrize("deterministic", [False, True])
def test_dropin_fused_step_matches_general_path(model, device, monkeypatch, deterministic):
    # The one-call decode step (append or block opening, table update and
    # decode launch in tierkv_decode_step) against the general path of three
    # calls: the same logits and HOT pool contents (to the decode kernel's
    # run-to-run rounding, which reaches the later tokens' K/V through the
    # hidden states; bit for bit with the deterministic tile hand-out), the
    # same tables, WARM pools (written by the prefill) and block cursors.
    print(f"[hf] drop-in fused decode step vs three calls, deterministic={deterministic}", flush=True)
    monkeypatch.setenv("TIERKV_DETERMINISTIC", "1" if deterministic else "0")
    ids = _tokens(1, device)
    kw = dict(hot_budget=3, policy_interval=10_000, policy_mode="hot_warm", attention_backend="triton")
    rt_f = _dropin_runtime(model, **kw)
    taken = []
    orig = rt_f.fused_decode_step

    def counted(*a, **k):
        out = orig(*a, **k)
        taken.append(out is not None)
        return out

    monkeypatch.setattr(rt_f, "fused_decode_step", counted)
    got = _teacher_forced(model, ids, rt_f.cache)
    monkeypatch.setenv("TIERKV_FUSED_STEP", "0")
    rt_g = _dropin_runtime(model, **kw)
    ref = _teacher_forced(model, ids, rt_g.cache)
    # Every decode layer-step but the first (whose table entries from the
    # prefill exceed the inline writes) takes the one-call path, the step
    # that opens the second decode block included.
    assert sum(taken) >= (STEPS - 1) * model.config.num_hidden_layers, taken
    pf, pg = rt_f.kv_pool, rt_g.kv_pool
    if deterministic:
        assert torch.equal(got, ref)
        assert torch.equal(pf.hot_k_pool, pg.hot_k_pool) and torch.equal(pf.hot_v_pool, pg.hot_v_pool)
    else:
        torch.testing.assert_close(got, ref, atol=2e-3, rtol=2e-3)
        torch.testing.assert_close(pf.hot_k_pool, pg.hot_k_pool, atol=2e-2, rtol=2e-2)
        torch.testing.assert_close(pf.hot_v_pool, pg.hot_v_pool, atol=2e-2, rtol=2e-2)
    for k in range(pf._tables.shape[1]):
        assert torch.equal(pf._tables.view(k), pg._tables.view(k))
    assert torch.equal(pf.warm_k_pool, pg.warm_k_pool) and torch.equal(pf.warm_v_pool, pg.warm_v_pool)
    for layer in range(model.config.num_hidden_layers):
        cf, cg = rt_f.layer_states[layer], rt_g.layer_states[layer]
        assert (cf.open_physical_idx, cf.open_token_count, cf.num_blocks) == \
            (cg.open_physical_idx, cg.open_token_count, cg.num_blocks)


def test_dropin_refused_step_keeps_tables_consistent(model, device, monkeypatch):
    """A one-call decode step that the library refuses (its checks run before
    its first launch, so nothing reached the device) leaves the drop-in's
    ledger, block cursor and tables as they were, with the step's table
    writes queued again: after a flush the device tables equal the host
    copies.  The same step then goes through."""
    from paged_tierkv_amd import _lib

    print("[hf] drop-in refused one-call step", flush=True)
    ids = _tokens(1, device)
    rt = _dropin_runtime(model, hot_budget=3, policy_interval=10_000, policy_mode="hot_warm",
                         attention_backend="triton")
    with torch.no_grad():
        out = model(input_ids=ids[:, :PROMPT], past_key_values=rt.cache, use_cache=True, logits_to_keep=1)
        for s in range(3):
            out = model(input_ids=ids[:, PROMPT + s: PROMPT + s + 1], past_key_values=out.past_key_values,
                        use_cache=True, logits_to_keep=1)
    cfg = model.config
    heads, kvh, dim = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    g = torch.Generator().manual_seed(3)
    q = torch.randn((1, heads, 1, dim), generator=g).half().to(device)
    k = torch.randn((1, kvh, 1, dim), generator=g).half().to(device)
    v = torch.randn((1, kvh, 1, dim), generator=g).half().to(device)
    pool, layer = rt.kv_pool, 0
    cursor = rt.layer_states[layer]
    assert cursor.open_physical_idx is not None
    before = (cursor.open_physical_idx, cursor.open_token_count, cursor.num_blocks)
    ledger = dict(pool._blocks)

    def tables_agree():
        for t in range(pool._tables.shape[1]):
            host = torch.from_numpy(pool._tables.host[:, t].copy())
            assert torch.equal(pool._tables.view(t).cpu(), host), t

    tables_agree()
    monkeypatch.setattr(_lib.lib(), "tierkv_decode_step", lambda *a: _lib.TIERKV_ERR_INVALID)
    with pytest.raises(ValueError):
        rt.fused_decode_step(layer, q, k, v, heads // kvh, dim ** -0.5)
    assert (cursor.open_physical_idx, cursor.open_token_count, cursor.num_blocks) == before
    assert pool._blocks == ledger
    tables_agree()
    monkeypatch.undo()
    out = rt.fused_decode_step(layer, q, k, v, heads // kvh, dim ** -0.5)
    assert out is not None and torch.isfinite(out.float()).all()
    assert cursor.open_token_count == before[1] + 1
    tables_agree()


def test_dropin_policy_ticks_run(model, device):
    print("[hf] drop-in hot_warm_cold with ticks", flush=True)
    ids = _tokens(1, device)
    rt = _dropin_runtime(model, hot_budget=3, attention_backend="triton", policy_interval=4,
                         policy_mode="hot_warm_cold", warm_budget=2)
    got = _teacher_forced(model, ids, rt.cache)
    assert torch.isfinite(got).all()
    m = rt.collect_memory_metrics()
    assert m["cold_blocks"] > 0 and m["warm_blocks"] > 0


def test_batched_all_hot_matches_stock(model, device):
    print("[hf] batched all-HOT vs stock", flush=True)
    from transformers import DynamicCache

    ids = _tokens(3, device)
    ref = _teacher_forced(model, ids, DynamicCache(config=model.config))
    cfg = model.config
    rt = BatchedTieredKVRuntime(cfg.num_hidden_layers, 3, cfg.num_key_value_heads, cfg.head_dim,
                                PROMPT + STEPS + 16, hot_fraction=1.0, warm_fraction=0.0, policy_mode="hot_warm",
                                policy_interval=8, device=device)
    got = _teacher_forced(model, ids, rt.cache)
    rt.check_errors()
    torch.testing.assert_close(got, ref, atol=2e-2, rtol=2e-2)
    assert rt.cache.get_seq_length() == PROMPT + STEPS


def test_batched_tiered_runs(model, device):
    print("[hf] batched hot_warm_cold with device ticks", flush=True)
    ids = _tokens(4, device)
    cfg = model.config
    rt = BatchedTieredKVRuntime(cfg.num_hidden_layers, 4, cfg.num_key_value_heads, cfg.head_dim,
                                PROMPT + STEPS + 16, hot_fraction=0.15, warm_fraction=0.55,
                                policy_mode="hot_warm_cold", policy_interval=8, device=device)
    got = _teacher_forced(model, ids, rt.cache)
    rt.check_errors()
    assert torch.isfinite(got).all()
    m = rt.memory_metrics()
    assert m["cold_blocks"] > 0 and m["compression_x"] > 1.0


def test_attention_prefill_scoring_changes_tiers(model, device):
    """prefill_scoring="attention" ranks prompt blocks by the prefill
    block-score kernel instead of the sink + recency proxy: the prompt's tier
    layout differs, the run stays finite, and the batched runtime accepts the
    same option."""
    print("[hf] attention prefill scoring", flush=True)
    ids = _tokens(1, device)
    layouts = {}
    for scoring in ("proxy", "attention"):
        rt = _dropin_runtime(model, hot_budget=3, attention_backend="triton", policy_interval=10_000,
                             policy_mode="hot_warm_cold", warm_budget=2, prefill_scoring=scoring)
        with torch.no_grad():
            out = model(input_ids=ids[:, :PROMPT], past_key_values=rt.cache, use_cache=True, logits_to_keep=1)
        assert torch.isfinite(out.logits).all()
        layouts[scoring] = [rt.block_manager.get_states(layer) for layer in range(model.config.num_hidden_layers)]
    assert layouts["proxy"] != layouts["attention"]
    cfg = model.config
    rt = BatchedTieredKVRuntime(cfg.num_hidden_layers, 2, cfg.num_key_value_heads, cfg.head_dim, PROMPT + STEPS + 16,
                                hot_fraction=0.2, warm_fraction=0.3, policy_mode="hot_warm_cold", policy_interval=8,
                                device=device, prefill_scoring="attention")
    got = _teacher_forced(model, _tokens(2, device), rt.cache)
    rt.check_errors()
    assert torch.isfinite(got).all()


def test_decode_graph_replays_match_eager(model, device):
    """Captured decode steps (two alternating graphs, eager policy steps in
    between) give the logits of the eager run, step by step, and leave the
    runtime in the same state."""
    print("[hf] decode graph runner vs eager", flush=True)
    cfg = model.config
    steps = 30
    ids = torch.randint(0, 1000, (3, PROMPT + steps), generator=torch.Generator().manual_seed(12)).to(device)

    def make():
        return BatchedTieredKVRuntime(cfg.num_hidden_layers, 3, cfg.num_key_value_heads, cfg.head_dim,
                                      PROMPT + steps + 16, hot_fraction=0.2, warm_fraction=0.4,
                                      policy_mode="hot_warm_cold", policy_interval=8, device=device)

    with torch.no_grad():
        rt_e = make()
        rt_e.fixed_launch_bound = True           # the same launches as the graphs
        model(input_ids=ids[:, :PROMPT], past_key_values=rt_e.cache, use_cache=True, logits_to_keep=1)
        ref = []
        for s in range(steps):
            out = model(input_ids=ids[:, PROMPT + s: PROMPT + s + 1], past_key_values=rt_e.cache, use_cache=True,
                        logits_to_keep=1)
            ref.append(out.logits[:, -1].float().clone())
        rt_g = make()
        model(input_ids=ids[:, :PROMPT], past_key_values=rt_g.cache, use_cache=True, logits_to_keep=1)
    runner = hf_llama.DecodeGraphRunner(model, rt_g)
    for s in range(steps):
        logits = runner.step(ids[:, PROMPT + s: PROMPT + s + 1])
        got = logits[:, -1].float()
        torch.cuda.synchronize()
        # The decode kernel hands tiles to waves dynamically, so two eager runs
        # already differ at the fp32 rounding level; compare at model tolerance.
        print(f"step {s}: max |diff| {(got - ref[s]).abs().max().item():.2e}", flush=True)
        torch.testing.assert_close(got, ref[s], atol=1e-2, rtol=1e-2)
    assert runner.replays > 10 and len(runner.graphs) == 2
    rt_e.check_errors()
    rt_g.check_errors()
    for le, lg in zip(rt_e.layers, rt_g.layers):
        for name in ("table", "states", "lengths", "nblocks", "open", "hot_free", "warm_free", "ctl"):
            assert torch.equal(getattr(le, name), getattr(lg, name)), name
    assert rt_g.cache.get_seq_length() == rt_e.cache.get_seq_length() == PROMPT + steps

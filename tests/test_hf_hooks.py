"""Host-side checks of the HF hooks (paged_tierkv_amd.hf_llama) that need no
GPU: the stock path is untouched after install(), the tiered cache object
speaks transformers' cache protocol (mask sizes, query offset), and the
prefill proxy scores have the reference's closed form
(modeling_llama.py:282-302)."""

from __future__ import annotations

import pytest
import torch

transformers = pytest.importorskip("transformers")

from paged_tierkv_amd import hf_llama  # noqa: E402
from paged_tierkv_amd.tierkv_policy import TieredKVCache  # noqa: E402


def _tiny_model():
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(hidden_size=64, intermediate_size=128, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=2, vocab_size=100, max_position_embeddings=256)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg).eval()


def test_stock_path_unchanged_after_install():
    model = _tiny_model()
    ids = torch.randint(0, 100, (2, 12), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        ref = model(input_ids=ids, use_cache=True)
        ref2 = model(input_ids=ids[:, :1], past_key_values=ref.past_key_values, use_cache=True)
    hf_llama.install()
    try:
        with torch.no_grad():
            got = model(input_ids=ids, use_cache=True)
            got2 = model(input_ids=ids[:, :1], past_key_values=got.past_key_values, use_cache=True)
    finally:
        hf_llama.uninstall()
    torch.testing.assert_close(got.logits, ref.logits, atol=0, rtol=0)
    torch.testing.assert_close(got2.logits, ref2.logits, atol=0, rtol=0)


class _StubRuntime:
    num_layers = 2

    def __init__(self):
        self.calls = []

    def begin_forward(self, q):
        self.calls.append(("begin", q))

    def finish_forward(self):
        self.calls.append(("finish",))


def test_tiered_cache_protocol_with_transformers_masks():
    from transformers.masking_utils import create_causal_mask

    model = _tiny_model()
    rt = _StubRuntime()
    cache = TieredKVCache(rt)
    cache.begin_forward(10)
    assert cache.get_seq_length() == 0 and cache.get_mask_sizes(10) == (10, 0)
    emb = torch.zeros(1, 10, 64)
    create_causal_mask(config=model.config, inputs_embeds=emb, attention_mask=torch.ones(1, 10, dtype=torch.long),
                       past_key_values=cache, position_ids=torch.arange(10)[None])
    cache.finish_forward()
    assert cache.get_seq_length() == 10 and cache.get_query_offset(0) == 10
    cache.begin_forward(1)
    assert cache.get_mask_sizes(1) == (11, 0)
    create_causal_mask(config=model.config, inputs_embeds=emb[:, :1], attention_mask=torch.ones(1, 11, dtype=torch.long),
                       past_key_values=cache, position_ids=torch.tensor([[10]]))
    cache.finish_forward()
    assert rt.calls == [("begin", 10), ("finish",), ("begin", 1), ("finish",)]
    assert len(cache) == 2 and cache.get_max_cache_shape() == -1 and not cache.is_compileable


def test_prefill_proxy_scores_closed_form():
    s = hf_llama.compute_prefill_block_scores(None, None, 5 * 16 + 3, 16, torch.device("cpu"))
    want = torch.tensor([1.0, 1 / 5, 2 / 5, 3 / 5, 4 / 5, 1.0], dtype=torch.float32)
    assert torch.equal(s, want)
    assert hf_llama.compute_prefill_block_scores(None, None, 7, 16, torch.device("cpu")).tolist() == [1.0]
    assert hf_llama.compute_prefill_block_scores(None, None, 0, 16, torch.device("cpu")).numel() == 0


def test_mask_safety_rule():
    assert hf_llama._is_tierkv_triton_mask_safe(None)
    assert hf_llama._is_tierkv_triton_mask_safe(torch.ones(1, 5))
    assert not hf_llama._is_tierkv_triton_mask_safe(torch.ones(1, 1, 5, 5))

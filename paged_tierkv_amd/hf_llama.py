"""HF Llama hooks of the tiered KV cache on MI355X.

The reference ships a modified copy of transformers' modeling_llama.py whose
TierKV parts are: the runtime lookup and mask check (modeling_llama.py:50-73),
the prefill score helpers (250-302), the tiered branch of
``LlamaAttention.forward`` (350-506) and the ``begin_forward`` /
``finish_forward`` bracket in ``LlamaModel.forward`` (612-651).  Here the same
behaviour is installed onto the installed transformers' own Llama classes
(``install()``), so no model file is copied:

* ``LlamaModel.forward`` picks the global runtime's cache when none is given,
  brackets the call with ``begin_forward`` / ``finish_forward`` and passes
  ``tierkv_triton_mask_safe`` down to the attention layers;
* ``LlamaAttention.forward`` keeps the stock path for every other cache and,
  for a tiered cache, runs the reference's prefill / decode sequence: append,
  attend, score, policy, with the decode attention in the HIP kernel
  (``tierkv_hip.tierkv_decode_attention``) and every pool operation in the
  runtime's HIP kernels.

Two runtimes plug in through their ``cache`` object:

* ``tierkv_policy.TieredKVRuntime`` -- the reference API (batch 1, one
  BlockManager sequence per layer), driven call for call as the reference
  hook drives it;
* ``runtime.BatchedTieredKVRuntime`` -- B sequences in lockstep
  (``is_batched``): prefill goes straight to the tiers, each decode step is
  one ``decode_layer`` call (fused append, attention, and on policy steps the
  device-side tick).  Sequences must be unpadded and of equal length, the
  same restriction the reference's decode path has (batch 1, no padding,
  modeling_llama.py:70-73).
"""

from __future__ import annotations

from typing import Callable

import torch

from .tierkv_hip import tierkv_decode_attention
from .tierkv_policy import get_global_tierkv_runtime

_ORIGINALS: dict = {}


def _is_tierkv_triton_mask_safe(attention_mask) -> bool:
    """modeling_llama.py:70-73: the decode kernel applies no mask, so only
    unpadded (2-D or absent) masks may take the kernel path."""
    if attention_mask is None:
        return True
    return attention_mask.ndim == 2


def compute_attention_score_proxy(module, query: torch.Tensor, key: torch.Tensor, attention_mask,
                                  scaling: float, query_chunk_size: int = 64) -> torch.Tensor:
    """Mean softmax probability per key token over (batch, heads, queries),
    [1, 1, 1, T] in the query dtype (modeling_llama.py:250-279).  Used only by
    the eager-backend policy path, which attends over reconstructed K/V with
    the model's own attention."""
    from transformers.models.llama.modeling_llama import repeat_kv

    key_states = repeat_kv(key, module.num_key_value_groups)
    token_score_sum = torch.zeros(key_states.shape[-2], device=query.device, dtype=torch.float32)
    score_count = 0
    for start in range(0, query.shape[-2], query_chunk_size):
        end = min(start + query_chunk_size, query.shape[-2])
        logits = torch.matmul(query[:, :, start:end, :], key_states.transpose(2, 3).contiguous()) * scaling
        if attention_mask is not None:
            mask = attention_mask
            if attention_mask.ndim >= 3:
                mask = attention_mask.narrow(attention_mask.ndim - 2, start, end - start)
            logits = logits + mask
        weights = torch.softmax(logits, dim=-1, dtype=torch.float32)
        token_score_sum += weights.sum(dim=(0, 1, 2))
        score_count += weights.shape[0] * weights.shape[1] * weights.shape[2]
    return (token_score_sum / max(score_count, 1)).to(query.dtype).view(1, 1, 1, -1)


def compute_prefill_block_scores(policy_engine, attn_weights, seq_len: int, block_size: int,
                                 device: torch.device) -> torch.Tensor:
    """Prefill block scores (modeling_llama.py:282-302): the block mass of the
    attention probabilities when the attention returned them, else the sink +
    recency proxy (block i scores i / (n - 1); first and last blocks 1)."""
    if attn_weights is not None:
        return policy_engine.compute_block_scores(attn_weights)
    num_blocks = (int(seq_len) + int(block_size) - 1) // int(block_size)
    if num_blocks <= 0:
        return torch.empty(0, device=device, dtype=torch.float32)
    scores = torch.arange(num_blocks, device=device, dtype=torch.float32)
    if num_blocks > 1:
        scores = scores / float(num_blocks - 1)
    scores[0] = 1.0
    scores[-1] = 1.0
    return scores


def _attention_interface(module):
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    from transformers.models.llama.modeling_llama import eager_attention_forward

    fn: Callable = ALL_ATTENTION_FUNCTIONS.get_interface(module.config._attn_implementation,
                                                          eager_attention_forward)
    return fn


def _attention_block_scores(runtime, query_states, key_states, scaling):
    """Per-sequence prefill block scores [B, n] from the prefill block-score
    kernel (no materialised probabilities), when the runtime asks for them
    (``prefill_scoring="attention"``); None otherwise."""
    if getattr(runtime, "prefill_scoring", "proxy") != "attention":
        return None
    from . import kernels

    return kernels.prefill_block_mass(query_states, key_states, runtime.block_size, scaling)


def _batched_block_scores(attn_weights, runtime, seq_len: int):
    """Per-sequence prefill scores [B, n] from returned probabilities
    [B, H, Q, T] (mean over heads and queries, then over the block's tokens,
    in the block-mass kernel), or None for the runtime's sink + recency proxy."""
    if attn_weights is None:
        return None
    from . import kernels

    b, h, q, t = attn_weights.shape
    bs = runtime.block_size
    n = (t + bs - 1) // bs
    probs = torch.zeros((b, h * q, n * bs), dtype=torch.float32, device=attn_weights.device)
    probs[:, :, :t].copy_(attn_weights.reshape(b, h * q, t))
    lengths = torch.full((b, n), bs, dtype=torch.int32)
    lengths[:, -1] = t - bs * (n - 1)
    return kernels.block_mass_from_probs(probs, bs, lengths)


def tierkv_attention_forward(self, hidden_states: torch.Tensor, position_embeddings=None, attention_mask=None,
                             past_key_values=None, **kwargs):
    """``LlamaAttention.forward`` with the tiered branch (modeling_llama.py:350-506)."""
    tiered = getattr(past_key_values, "is_tierkv_cache", False)
    runtime = getattr(past_key_values, "runtime", None) if tiered else get_global_tierkv_runtime()
    if runtime is None or not tiered:
        return _ORIGINALS["attention"](self, hidden_states, position_embeddings, attention_mask, past_key_values,
                                       **kwargs)
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

    input_shape = hidden_states.shape[:-1]
    hidden_shape = (*input_shape, -1, self.head_dim)
    query_states = self.q_proj(hidden_states).view(hidden_shape).transpose(1, 2)
    key_states = self.k_proj(hidden_states).view(hidden_shape).transpose(1, 2)
    value_states = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
    cos, sin = position_embeddings
    dropout = 0.0 if not self.training else self.attention_dropout
    if (getattr(runtime, "is_batched", False) and getattr(runtime, "fused_rope", False)
            and query_states.shape[-2] == 1 and query_states.dtype == torch.float16
            and cos.dtype == torch.float16 and bool(kwargs.get("tierkv_triton_mask_safe", False))):
        # Decode step: the append kernel applies the rotation (same fp16 ops).
        out = runtime.decode_layer(self.layer_idx, query_states, key_states, value_states, self.num_key_value_groups,
                                   self.scaling, policy_step=runtime.policy_tick_this_forward, rope=(cos, sin))
        return self.o_proj(out.reshape(*input_shape, -1)), None
    query_states, key_states = apply_rotary_pos_emb(query_states, key_states, cos, sin)

    if getattr(runtime, "is_batched", False):
        return _batched_forward(self, runtime, query_states, key_states, value_states, attention_mask,
                                input_shape, dropout, kwargs)

    seq_id = self.layer_idx
    query_len = query_states.shape[-2]
    decode_total_start = runtime.profile_start() if query_len == 1 else None
    if query_len > 1:
        start = runtime.profile_start()
        attn_output, attn_weights = _attention_interface(self)(
            self, query_states, key_states, value_states, attention_mask, scaling=self.scaling, dropout=dropout)
        runtime.profile_end("prefill_attention_ms", start)
        if seq_id in runtime.tiered_layer_indices and runtime.policy_mode != "hot_only":
            start = runtime.profile_start()
            block_scores = None
            if attn_weights is None:
                block_scores = _attention_block_scores(runtime, query_states, key_states, self.scaling)
            if block_scores is not None:
                block_scores = block_scores[0]
            else:
                block_scores = compute_prefill_block_scores(runtime.policy_engine, attn_weights, key_states.shape[-2],
                                                            runtime.block_size, query_states.device)
            runtime.append_prefill_with_policy(seq_id, key_states, value_states, block_scores)
            runtime.profile_end("prefill_policy_ms", start)
        else:
            start = runtime.profile_start()
            runtime.append_to_layer(seq_id, key_states, value_states)
            runtime.profile_end("prefill_kv_append_ms", start)
        attn_output = attn_output.reshape(*input_shape, -1).contiguous()
        return self.o_proj(attn_output), attn_weights

    output_attentions = bool(kwargs.get("output_attentions", False))
    mask_safe = bool(kwargs.get("tierkv_triton_mask_safe", False))
    if runtime.attention_backend == "triton" and not output_attentions and mask_safe and query_states.is_cuda:
        # The plain decode step (token into the open HOT block, no policy, no
        # scores): append, table and decode in one C call.
        out = runtime.fused_decode_step(seq_id, query_states, key_states, value_states, self.num_key_value_groups,
                                        self.scaling)
        if out is not None:
            attn_output = self.o_proj(out.reshape(*input_shape, -1).contiguous())
            runtime.profile_end("decode_total_ms", decode_total_start)
            return attn_output, None
    start = runtime.profile_start()
    allocated_new_block = runtime.append_to_layer(seq_id, key_states, value_states)
    runtime.profile_end("decode_kv_append_ms", start)
    run_policy = runtime.should_run_decode_policy(seq_id, allocated_new_block)
    collect_scores = runtime.should_collect_decode_scores(seq_id, run_policy)
    use_kernel = (runtime.attention_backend == "triton" and not output_attentions and mask_safe
                  and query_states.is_cuda)
    if use_kernel:
        block_table, block_states, block_lengths, num_blocks = runtime.get_layer_table(seq_id)
        pool = runtime.kv_pool
        start = runtime.profile_start()
        attn_output, score_sums = tierkv_decode_attention(
            query_states, block_table, block_states, block_lengths, pool.hot_k_pool, pool.hot_v_pool,
            pool.warm_k_pool, pool.warm_v_pool, pool.k_scale, pool.k_zero, pool.v_scale, pool.v_zero,
            num_blocks=num_blocks, num_key_value_groups=self.num_key_value_groups, scaling=self.scaling,
            return_scores=collect_scores)
        runtime.profile_end("triton_decode_ms", start)
        attn_weights = None
        if collect_scores and score_sums is not None:
            start = runtime.profile_start()
            block_scores = runtime.block_scores_from_probability_sums(seq_id, score_sums)
            runtime.profile_end("decode_score_accum_ms", start)
            if run_policy:
                start = runtime.profile_start()
                runtime.enforce_policy(seq_id, block_scores)
                runtime.sync_storage_states(seq_id)
                runtime.profile_end("decode_policy_ms", start)
    else:
        start = runtime.profile_start()
        full_k, full_v, _, _ = runtime.reconstruct_layer(seq_id, allow_decode_reconstruct=True)
        runtime.profile_end("decode_reconstruct_ms", start)
        if full_k is None or full_v is None:
            raise RuntimeError(f"TieredKV failed to reconstruct KV tensors for layer {self.layer_idx}.")
        attn_output, attn_weights = _attention_interface(self)(
            self, query_states, full_k, full_v, attention_mask, scaling=self.scaling, dropout=dropout)
        if run_policy:
            start = runtime.profile_start()
            proxy = compute_attention_score_proxy(self, query_states, full_k, attention_mask, scaling=self.scaling)
            block_scores = runtime.policy_engine.compute_block_scores(proxy)
            runtime.enforce_policy(seq_id, block_scores)
            runtime.sync_storage_states(seq_id)
            runtime.profile_end("decode_policy_ms", start)
    attn_output = attn_output.reshape(*input_shape, -1).contiguous()
    attn_output = self.o_proj(attn_output)
    runtime.profile_end("decode_total_ms", decode_total_start)
    return attn_output, attn_weights


def _batched_forward(self, runtime, query_states, key_states, value_states, attention_mask, input_shape, dropout,
                     kwargs):
    layer = self.layer_idx
    if query_states.shape[-2] > 1:
        attn_output, attn_weights = _attention_interface(self)(
            self, query_states, key_states, value_states, attention_mask, scaling=self.scaling, dropout=dropout)
        scores = _batched_block_scores(attn_weights, runtime, key_states.shape[-2])
        if scores is None:
            scores = _attention_block_scores(runtime, query_states, key_states, self.scaling)
        runtime.prefill_layer(layer, key_states, value_states, block_scores=scores)
        attn_output = attn_output.reshape(*input_shape, -1).contiguous()
        return self.o_proj(attn_output), attn_weights
    if not bool(kwargs.get("tierkv_triton_mask_safe", False)):
        raise ValueError("the batched tiered runtime decodes unpadded sequences only (2-D or no attention mask).")
    out = runtime.decode_layer(layer, query_states, key_states, value_states, self.num_key_value_groups,
                               self.scaling, policy_step=runtime.policy_tick_this_forward)
    attn_output = out.reshape(*input_shape, -1)
    return self.o_proj(attn_output), None


def tierkv_model_forward(self, input_ids=None, attention_mask=None, position_ids=None, past_key_values=None,
                         inputs_embeds=None, use_cache=None, **kwargs):
    """``LlamaModel.forward`` bracketed for a tiered cache (modeling_llama.py:612-651)."""
    use = use_cache if use_cache is not None else getattr(self.config, "use_cache", False)
    if use and past_key_values is None:
        runtime = get_global_tierkv_runtime()
        if runtime is not None:
            past_key_values = runtime.cache
    tiered = bool(use) and getattr(past_key_values, "is_tierkv_cache", False)
    if tiered:
        query_length = (inputs_embeds if inputs_embeds is not None else input_ids).shape[1]
        past_key_values.begin_forward(query_length)
        kwargs["tierkv_triton_mask_safe"] = _is_tierkv_triton_mask_safe(attention_mask)
    out = _ORIGINALS["model"](self, input_ids=input_ids, attention_mask=attention_mask, position_ids=position_ids,
                              past_key_values=past_key_values, inputs_embeds=inputs_embeds, use_cache=use_cache,
                              **kwargs)
    if tiered:
        past_key_values.finish_forward()
    return out


class DecodeGraphRunner:
    """Decode steps of an HF Llama over a ``BatchedTieredKVRuntime`` replayed
    as HIP graphs.

    Between policy ticks a decode step launches the same kernels with the same
    arguments every time: the runtime's tables, free stacks and block counts
    live on the device, and the decode kernel is launched with the table width
    as its bound (``fixed_launch_bound``).  The step is therefore captured once
    and replayed, which removes the host cost of transformers' ~40 launches per
    layer.  The host bookkeeping a Python forward would do (step counter,
    block counts, cache length) is done by the runner around each replay.

    * The runtime's decode workspace is reserved here, at its largest size
      (``max_blocks`` with score sums), before anything is captured: captured
      launches and eager policy steps use that one buffer, which is never
      replaced.
    * The first step runs eagerly; the next two are captured and replayed.
      Policy steps run eagerly.
    * Two graphs alternate, so the logits a step returns stay valid while
      the next step is replayed.
    * ``step`` returns the graph's static logits tensor: read it before the
      same graph is replayed again (two steps later).
    * Everything runs on the current stream; sequences must be unpadded.
    """

    def __init__(self, model, runtime):
        if not getattr(runtime, "is_batched", False):
            raise ValueError("DecodeGraphRunner drives a BatchedTieredKVRuntime.")
        self.model = model
        self.rt = runtime
        runtime.fixed_launch_bound = True
        runtime.reserve_decode_workspace(model.config.num_attention_heads)
        self.ids = torch.zeros((runtime.batch, 1), dtype=torch.long, device=runtime.device)
        self.pos = torch.zeros((1, 1), dtype=torch.long, device=runtime.device)
        self.graphs: list = []
        self.outs: list = []
        self.turn = 0
        self.eager_steps = 0
        self.replays = 0

    def _forward(self):
        return self.model(input_ids=self.ids, position_ids=self.pos, past_key_values=self.rt.cache, use_cache=True,
                          logits_to_keep=1).logits

    def step(self, input_ids: torch.Tensor) -> torch.Tensor:
        """One decode step for input_ids [B, 1]; returns logits [B, 1, V]."""
        rt = self.rt
        self.ids.copy_(input_ids)
        self.pos.fill_(rt.cache.get_seq_length())
        tick_next = (rt.decode_step + 1) % rt.policy_interval == 0
        with torch.no_grad():
            if tick_next or self.eager_steps == 0:
                self.eager_steps += 1
                return self._forward()
            if len(self.graphs) < 2:
                # The Python forward runs once under capture (doing this step's
                # host bookkeeping); the recorded kernels then run by replay.
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    out = self._forward()
                self.graphs.append(g)
                self.outs.append(out)
                g.replay()
                self.turn = len(self.graphs) % 2
                return out
        g, out = self.graphs[self.turn], self.outs[self.turn]
        self.turn ^= 1
        rt.cache.begin_forward(1)
        for layer in range(rt.num_layers):
            rt._advance_blocks(layer, 1)
        g.replay()
        rt.cache.finish_forward()
        self.replays += 1
        return out


def install() -> None:
    """Patch the installed transformers' LlamaAttention / LlamaModel forwards
    (idempotent).  Models without a tiered cache keep the stock behaviour."""
    from transformers.models.llama import modeling_llama as ml

    if "attention" not in _ORIGINALS:
        _ORIGINALS["attention"] = ml.LlamaAttention.forward
        _ORIGINALS["model"] = ml.LlamaModel.forward
    ml.LlamaAttention.forward = tierkv_attention_forward
    ml.LlamaModel.forward = tierkv_model_forward


def uninstall() -> None:
    from transformers.models.llama import modeling_llama as ml

    if "attention" in _ORIGINALS:
        ml.LlamaAttention.forward = _ORIGINALS.pop("attention")
        ml.LlamaModel.forward = _ORIGINALS.pop("model")

"""Seeded synthetic inputs for the BASELINE configurations.

Every tensor is generated on the CPU with a seeded ``torch.Generator`` so
the HIP path and the CPU oracle see identical bits; callers move what they
need to the GPU.  WARM tiles are returned as fp16 *sources*
(``warm_src_k/v``); the caller quantizes them (the HIP demotion kernel on the
GPU, or the oracle codec on the CPU).

Configs (BASELINE.json ``configs``):

* C1 -- TinyLlama shape: 32 q / 4 kv heads, head_dim 64, batch 1, 512
  tokens = 32 blocks of 16; 8 HOT / 16 WARM / 8 COLD; block 0 always HOT,
  the rest by seeded shuffle; first 4 tokens x4; dense layout: physical ids
  are the first 32 entries of a random permutation of a 64-block pool.
* C2(a) -- demotion: 4096-block fp16 pools [4096, 8, 16, 128] (K and V),
  a seeded 50 % of the logical blocks demoted in ascending order.
* C2(b) -- scoring: probabilities softmax(3 * N(0, 1)) [32, 32, 4096].
* C3 -- Llama-3-8B shape: 32 q / 8 kv heads, head_dim 128, batch 32, 4096
  tokens = 256 blocks; per sequence 26 HOT (block 0, the last 8 and 17 by
  shuffle) / 154 WARM / 76 COLD; compact layout with slots shuffled across
  shared pools.
* C4 -- as C3 with batch 4 and 32768 tokens = 2048 blocks; 102 HOT / 922
  WARM / 1024 COLD; first 4 tokens x4 and a seeded 2 % of blocks x2.

Tier counts use round-half-even fractions with COLD as the remainder.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

HOT, WARM, COLD = 0, 1, 2

CONFIG_SEEDS = {"c1": 1, "c2a": 2, "c2b": 3, "c3": 4, "c4": 5}


@dataclass
class TieredDecodeCase:
    name: str
    batch: int
    num_heads: int
    kv_heads: int
    head_dim: int
    block_size: int
    num_blocks: int
    query: torch.Tensor            # fp16 [B, H, 1, D]
    block_table: torch.Tensor      # int32 [B, maxB]
    block_states: torch.Tensor     # int32 [B, maxB]
    block_lengths: torch.Tensor    # int32 [B, maxB]
    hot_k: torch.Tensor            # fp16 [S_hot, H_kv, bs, D]
    hot_v: torch.Tensor
    warm_src_k: torch.Tensor       # fp16 [S_warm, H_kv, bs, D] before quantization
    warm_src_v: torch.Tensor
    cold_mode: str = "masked"
    layout: str = "compact"
    seed: int = 0
    meta: dict = field(default_factory=dict)

    @property
    def groups(self) -> int:
        return self.num_heads // self.kv_heads

    @property
    def scaling(self) -> float:
        return self.head_dim ** -0.5

    def tier_counts(self):
        s = self.block_states[:, : self.num_blocks]
        return [(int((row == HOT).sum()), int((row == WARM).sum()), int((row == COLD).sum())) for row in s]


def tier_split(num_blocks: int, hot_frac: float, warm_frac: float):
    """Round-half-even tier counts, COLD as the remainder."""
    n_hot = int(round(num_blocks * hot_frac))
    n_warm = int(round(num_blocks * warm_frac))
    return n_hot, n_warm, num_blocks - n_hot - n_warm


def assign_tiers(gen, num_blocks, n_hot, n_warm, always_hot):
    """Per-sequence states: ``always_hot`` blocks first, then a seeded
    shuffle of the others fills the rest of HOT, then WARM, then COLD."""
    always = sorted(set(int(i) for i in always_hot if 0 <= i < num_blocks))
    states = torch.full((num_blocks,), COLD, dtype=torch.int32)
    states[always] = HOT
    rest = torch.tensor([i for i in range(num_blocks) if i not in set(always)], dtype=torch.long)
    order = rest[torch.randperm(len(rest), generator=gen)]
    extra_hot = max(n_hot - len(always), 0)
    states[order[:extra_hot]] = HOT
    states[order[extra_hot: extra_hot + n_warm]] = WARM
    return states


def _randn_f16(gen, shape):
    return torch.randn(shape, generator=gen, dtype=torch.float32).to(torch.float16)


def make_tiered_case(name, batch, num_heads, kv_heads, head_dim, num_blocks, n_hot, n_warm, seed,
                     block_size=16, recent_hot=0, layout="compact", dense_pool_blocks=None,
                     sink_tokens=0, sink_scale=4.0, heavy_frac=0.0, heavy_scale=2.0,
                     lengths=None, cold_mode="masked", max_blocks=None, with_data=True):
    """General tiered-decode generator (see module docstring for presets).

    lengths: None (all blocks full) or int32 [B, num_blocks] valid-token
    counts.  layout "compact": tables hold state-specific slots (COLD -1);
    "dense": tables hold physical ids that index both pools.  with_data=False
    returns only the metadata (pools are empty [0, ...] tensors; the
    ``meta`` dict holds the slot counts) for callers that fill pools on the
    GPU."""
    gen = torch.Generator().manual_seed(int(seed))
    max_blocks = int(max_blocks or num_blocks)
    states = torch.full((batch, max_blocks), COLD, dtype=torch.int32)
    always = [0] + list(range(num_blocks - recent_hot, num_blocks))
    for b in range(batch):
        states[b, :num_blocks] = assign_tiers(gen, num_blocks, n_hot, n_warm, always)
    lens = torch.zeros((batch, max_blocks), dtype=torch.int32)
    if lengths is None:
        lens[:, :num_blocks] = block_size
    else:
        lens[:, :num_blocks] = torch.as_tensor(lengths, dtype=torch.int32)
    table = torch.full((batch, max_blocks), -1, dtype=torch.int32)
    active = states[:, :num_blocks]
    if layout == "dense":
        pool = int(dense_pool_blocks or batch * num_blocks)
        perm = torch.randperm(pool, generator=gen)[: batch * num_blocks].view(batch, num_blocks)
        table[:, :num_blocks] = perm.to(torch.int32)
        n_hot_slots = n_warm_slots = pool
        hot_slot_of = {(b, i): int(perm[b, i]) for b in range(batch) for i in range(num_blocks) if active[b, i] == HOT}
        warm_slot_of = {(b, i): int(perm[b, i]) for b in range(batch) for i in range(num_blocks) if active[b, i] == WARM}
    else:
        hot_pos = [(b, i) for b in range(batch) for i in range(num_blocks) if active[b, i] == HOT]
        warm_pos = [(b, i) for b in range(batch) for i in range(num_blocks) if active[b, i] == WARM]
        hp = torch.randperm(max(len(hot_pos), 1), generator=gen).tolist()
        wp = torch.randperm(max(len(warm_pos), 1), generator=gen).tolist()
        hot_slot_of = {pos: hp[k] for k, pos in enumerate(hot_pos)}
        warm_slot_of = {pos: wp[k] for k, pos in enumerate(warm_pos)}
        n_hot_slots = max(len(hot_pos), 1)
        n_warm_slots = max(len(warm_pos), 1)
        for (b, i), s in hot_slot_of.items():
            table[b, i] = s
        for (b, i), s in warm_slot_of.items():
            table[b, i] = s

    shape_h = (n_hot_slots, kv_heads, block_size, head_dim)
    shape_w = (n_warm_slots, kv_heads, block_size, head_dim)
    if not with_data:
        empty = torch.empty((0, kv_heads, block_size, head_dim), dtype=torch.float16)
        return TieredDecodeCase(
            name=name, batch=batch, num_heads=num_heads, kv_heads=kv_heads, head_dim=head_dim,
            block_size=block_size, num_blocks=num_blocks,
            query=_randn_f16(gen, (batch, num_heads, 1, head_dim)), block_table=table,
            block_states=states, block_lengths=lens, hot_k=empty, hot_v=empty, warm_src_k=empty,
            warm_src_v=empty, cold_mode=cold_mode, layout=layout, seed=int(seed),
            meta={"n_hot": n_hot, "n_warm": n_warm, "hot_slots": n_hot_slots, "warm_slots": n_warm_slots})
    hot_k, hot_v = _randn_f16(gen, shape_h), _randn_f16(gen, shape_h)
    warm_k, warm_v = _randn_f16(gen, shape_w), _randn_f16(gen, shape_w)
    query = _randn_f16(gen, (batch, num_heads, 1, head_dim))

    # Sink tokens (first tokens of logical block 0) and heavy-hitter blocks.
    heavy = torch.zeros((batch, num_blocks), dtype=torch.bool)
    if heavy_frac > 0:
        heavy = torch.rand((batch, num_blocks), generator=gen) < heavy_frac
    for pool_k, pool_v, slot_of in ((hot_k, hot_v, hot_slot_of), (warm_k, warm_v, warm_slot_of)):
        for (b, i), s in slot_of.items():
            f = heavy_scale if heavy[b, i] else 1.0
            if i == 0 and sink_tokens > 0:
                pool_k[s, :, :sink_tokens] = (pool_k[s, :, :sink_tokens].float() * sink_scale).half()
                pool_v[s, :, :sink_tokens] = (pool_v[s, :, :sink_tokens].float() * sink_scale).half()
            if f != 1.0:
                pool_k[s] = (pool_k[s].float() * f).half()
                pool_v[s] = (pool_v[s].float() * f).half()

    return TieredDecodeCase(
        name=name, batch=batch, num_heads=num_heads, kv_heads=kv_heads, head_dim=head_dim,
        block_size=block_size, num_blocks=num_blocks, query=query, block_table=table,
        block_states=states, block_lengths=lens, hot_k=hot_k, hot_v=hot_v,
        warm_src_k=warm_k, warm_src_v=warm_v, cold_mode=cold_mode, layout=layout, seed=int(seed),
        meta={"n_hot": n_hot, "n_warm": n_warm, "heavy_blocks": int(heavy.sum())})


def config1(seed=None):
    return make_tiered_case("c1_tinyllama_b1_ctx512", 1, 32, 4, 64, 32, 8, 16,
                            seed=CONFIG_SEEDS["c1"] if seed is None else seed,
                            layout="dense", dense_pool_blocks=64, sink_tokens=4)


def config3(seed=None, batch=32, with_data=True):
    n_hot, n_warm, _ = tier_split(256, 0.10, 0.60)
    return make_tiered_case("c3_llama3_8b_b32_ctx4096", batch, 32, 8, 128, 256, n_hot, n_warm,
                            seed=CONFIG_SEEDS["c3"] if seed is None else seed, recent_hot=8,
                            with_data=with_data)


def config4(seed=None, batch=4, with_data=True):
    n_hot, n_warm, _ = tier_split(2048, 0.05, 0.45)
    return make_tiered_case("c4_llama3_8b_b4_ctx32768", batch, 32, 8, 128, 2048, n_hot, n_warm,
                            seed=CONFIG_SEEDS["c4"] if seed is None else seed, recent_hot=8,
                            sink_tokens=4, heavy_frac=0.02, with_data=with_data)


def ideal_bytes(states, num_blocks, num_heads, kv_heads, head_dim, block_size=16, warm_format="absmax_i8",
                return_scores=False):
    """Algorithmic HBM bytes of one decode launch over ``states`` [B, maxB]:
    per sequence HOT blocks 2*H_kv*bs*D*2 (K+V fp16), WARM blocks
    2*H_kv*bs*D (int8 codes) + metadata (absmax 2*H_kv*4 B; reference
    format 2*2*H_kv*bs*2 B), COLD 0, 12 B of table/state/length per block,
    2*H*D*2 B of query in and output out; scores add H*n_blocks*4."""
    st = torch.as_tensor(states)[:, :num_blocks]
    n_hot = int((st == HOT).sum())
    n_warm = int((st == WARM).sum())
    meta = 2 * kv_heads * 4 if warm_format == "absmax_i8" else 2 * 2 * kv_heads * block_size * 2
    b = st.shape[0]
    total = n_hot * 2 * kv_heads * block_size * head_dim * 2
    total += n_warm * (2 * kv_heads * block_size * head_dim + meta)
    total += b * (num_blocks * 12 + 2 * num_heads * head_dim * 2)
    if return_scores:
        total += b * num_heads * num_blocks * 4
    return total


@dataclass
class DemoteCase:
    hot_k: torch.Tensor       # fp16 [4096, 8, 16, 128]
    hot_v: torch.Tensor
    table: torch.Tensor       # int32 [1, 4096]  logical -> hot slot
    states: torch.Tensor      # int32 [1, 4096]  all HOT
    demote_logical: torch.Tensor   # int64 sorted logical ids to demote
    warm_slots: torch.Tensor  # int32 warm slot per demoted block (prefix-sum order)


def config2a(seed=None, pool_blocks=4096, kv_heads=8, head_dim=128, block_size=16, frac=0.5):
    gen = torch.Generator().manual_seed(CONFIG_SEEDS["c2a"] if seed is None else int(seed))
    shape = (pool_blocks, kv_heads, block_size, head_dim)
    hot_k, hot_v = _randn_f16(gen, shape), _randn_f16(gen, shape)
    table = torch.randperm(pool_blocks, generator=gen).to(torch.int32).view(1, -1)
    states = torch.zeros((1, pool_blocks), dtype=torch.int32)
    n = int(round(pool_blocks * frac))
    demote = torch.randperm(pool_blocks, generator=gen)[:n].sort().values
    return DemoteCase(hot_k, hot_v, table, states, demote, torch.arange(n, dtype=torch.int32))


def config2b(seed=None, batch=32, heads=32, tokens=4096, logit_std=3.0):
    gen = torch.Generator().manual_seed(CONFIG_SEEDS["c2b"] if seed is None else int(seed))
    logits = torch.randn((batch, heads, tokens), generator=gen, dtype=torch.float32) * logit_std
    return torch.softmax(logits, dim=-1)


def demote_ideal_bytes(n_blocks, kv_heads, block_size, head_dim):
    """Algorithmic bytes of demoting n_blocks full blocks (K and V) to int8
    absmax: fp16 tiles read, int8 codes and fp32 per-(block, head) scales
    written, four int32 job-list entries read and two table entries
    (slot, state) written per block."""
    tile = kv_heads * block_size * head_dim
    return n_blocks * (2 * tile * 2 + 2 * tile + 2 * kv_heads * 4 + 4 * 4 + 2 * 4)


def codec_ideal_bytes(n_blocks, kv_heads, block_size, head_dim, warm_format="absmax_i8", op="demote"):
    """Algorithmic bytes of one demotion or promotion launch over n_blocks
    full blocks (K and V): the fp16 tiles, the 1-byte codes, the codec's
    metadata (absmax: one fp32 scale per (block, head); reference: fp16 scale
    and zero point per (token, head)), four int32 job-list entries read and
    two table entries (slot, state) written per block.  Demotion reads the
    fp16 tiles and writes codes and metadata; promotion the reverse."""
    tile = kv_heads * block_size * head_dim
    meta = 2 * kv_heads * 4 if warm_format == "absmax_i8" else 2 * 2 * kv_heads * block_size * 2
    return n_blocks * (2 * tile * 2 + 2 * tile + meta + 4 * 4 + 2 * 4)


def score_ideal_bytes(batch, heads, tokens, block_size):
    """Algorithmic bytes of one scoring step: fp32 probabilities read, fp32
    block mass written, then mass and current states read and labels
    written by the label kernel."""
    nblk = tokens // block_size
    return batch * heads * tokens * 4 + batch * nblk * 4 + batch * nblk * (4 + 4 + 4)


C2B_HOT_BUDGET = 26     # block 0 and 255 plus 24 by score
C2B_COLD_COUNT = 77
C2B_WARM_BUDGET = 256 - C2B_HOT_BUDGET - C2B_COLD_COUNT


def llama3_8b_random(device, num_layers: int = 32):
    """Random-init Llama-3-8B-shaped decoder:
    32 layers, hidden 4096, 32 / 8 heads, head_dim 128, FFN 14336, vocab
    128256, fp16 weights ~N(0, 0.02) (transformers' own init with
    initializer_range 0.02), built directly on ``device``."""
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(hidden_size=4096, intermediate_size=14336, num_hidden_layers=num_layers,
                      num_attention_heads=32, num_key_value_heads=8, head_dim=128, vocab_size=128256,
                      max_position_embeddings=8192, rope_theta=500000.0, initializer_range=0.02,
                      rms_norm_eps=1e-5, tie_word_embeddings=False)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float16)
    try:
        with torch.device(device):
            model = LlamaForCausalLM(cfg).eval()
    finally:
        torch.set_default_dtype(prev)
    return model

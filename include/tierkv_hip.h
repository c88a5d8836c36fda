/*
 * tierkv_hip.h -- C ABI of the MI355X (gfx950) tiered paged KV-cache path.
 *
 * Plain pointers and sizes only: device pointers for tensors, a hipStream_t
 * passed as void*, int status codes.  Every launch is asynchronous on the
 * given stream and never synchronises.  The library keeps no pointer past a
 * call.  Citations are file:line in xiaoMartintin/Paged_TierKV.
 *
 * Tier states: 0 HOT (fp16), 1 WARM (quantized), 2 COLD (evicted)
 * (tierkv_policy.py:14-16, csrc/block_manager.cpp:9-13).
 *
 * Pool layouts (tierkv_policy.py:122-135, 828-841):
 *   hot_k/hot_v   fp16  [hot_slots,  kv_heads, block_size, head_dim]
 *   warm_k/warm_v       [warm_slots, kv_heads, block_size, head_dim]
 *     TIERKV_WARM_REF_U8:    uint8 codes, k/v_scale and k/v_zero fp16
 *                            [warm_slots, kv_heads, block_size, 1]
 *                            (quantize_fp16_to_int8, tierkv_policy.py:21-36)
 *     TIERKV_WARM_ABSMAX_I8: int8 codes, k/v_scale fp32 [warm_slots, kv_heads],
 *                            k/v_zero unused (NULL)
 *   block_table / block_states / block_lengths: int32 [batch, table_stride],
 *     indexed by logical block; the table holds the slot of the block's
 *     state-specific pool (compact layout) or a physical id that indexes both
 *     pools (dense layout); COLD entries are never dereferenced.
 */
#ifndef TIERKV_HIP_H
#define TIERKV_HIP_H

#include <stdint.h>

#if defined(__GNUC__)
#define TIERKV_API __attribute__((visibility("default")))
#else
#define TIERKV_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes (the Python layer maps 1 -> ValueError, others -> RuntimeError). */
#define TIERKV_OK 0
#define TIERKV_ERR_INVALID 1     /* bad argument / shape */
#define TIERKV_ERR_UNSUPPORTED 2 /* configuration outside the kernels' support */
#define TIERKV_ERR_HIP 3         /* HIP launch/runtime error */
#define TIERKV_ERR_WORKSPACE 4   /* workspace too small */
#define TIERKV_ERR_STATE 5       /* BlockManager rule violation (RuntimeError) */

#define TIERKV_DTYPE_F16 0
#define TIERKV_DTYPE_BF16 1

#define TIERKV_WARM_REF_U8 0
#define TIERKV_WARM_ABSMAX_I8 1

#define TIERKV_COLD_ZERO_LOGIT 0 /* reference: COLD tokens enter softmax with K=V=0 */
#define TIERKV_COLD_MASKED 1     /* COLD blocks contribute nothing */

/* Flag OR'ed into a decode call's splits_hint (whose low bits are the split
 * factor, 0 = automatic): each wave takes a fixed share of the workgroup's
 * tiles instead of taking them from a shared counter, so the attention output
 * is the same bits on every call over the same inputs, as the reference's
 * Triton kernel is.  Costs about 1 % of the launch time (2-3 % with score
 * sums). */
#define TIERKV_DECODE_DETERMINISTIC 0x40000000

/* Message of the last failing call on this thread ("" if none). */
TIERKV_API const char* tierkv_last_error(void);

/* Library/ABI version, for the Python loader's compatibility check. */
TIERKV_API int32_t tierkv_abi_version(void);

/* ---------------------------------------------------------------------- */
/* Decode attention.  Replaces the launch in tierkv_decode_attention
 * (tierkv_triton.py:272-465) of _tierkv_decode_attention_kernel
 * (tierkv_triton.py:45-145) and the split/reduce pair (147-264).
 *
 * query  [batch, num_heads, head_dim] (== [B, H, 1, D] contiguous), f16/bf16.
 * out    [batch, num_heads, head_dim] (== [B, 1, H, D]), same dtype as query.
 * score_sums  NULL, or fp32 [batch, num_heads, table_stride]: per (head,
 *   block) sum of softmax probabilities (tierkv_triton.py:121-145), zero for
 *   blocks >= the sequence's block count.
 * seq_num_blocks  NULL (every sequence has num_blocks blocks) or device
 *   int32 [batch] (each clamped to num_blocks).
 * workspace  device scratch of at least tierkv_decode_workspace_bytes(...)
 *   bytes, zero-filled before its first use; its first 4 bytes are an error
 *   word the kernels set non-zero when they skip a block whose slot or state
 *   is out of range.  It also holds the split-arrival counters, which every
 *   launch leaves at zero, so one workspace serves launches of any shape
 *   (and graph replays) on one stream; launches that share it must not
 *   overlap.
 * scaling  softmax scale (head_dim ** -0.5 in modeling_llama.py:315).
 * splits_hint  split factor per (sequence, kv head) (0: chosen from the
 *   launch size), optionally | TIERKV_DECODE_DETERMINISTIC.  Without the
 *   flag, tiles are handed to waves as they free up: outputs agree with the
 *   fp32 reference within tolerance but their last bits can differ between
 *   calls.  Score sums are the same bits either way.
 */
TIERKV_API int32_t tierkv_decode_attention(
    const void* query, int32_t query_dtype, void* out, float* score_sums,
    const int32_t* block_table, const int32_t* block_states, const int32_t* block_lengths,
    int64_t table_stride, const int32_t* seq_num_blocks, int32_t num_blocks,
    const void* hot_k, const void* hot_v, int64_t hot_slots,
    const void* warm_k, const void* warm_v, int64_t warm_slots,
    const void* k_scale, const void* k_zero, const void* v_scale, const void* v_zero,
    int32_t warm_format, int32_t cold_mode,
    int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t block_size, int32_t head_dim,
    float scaling, int32_t splits_hint,
    void* workspace, int64_t workspace_bytes, void* stream);

/* tierkv_decode_attention without a workspace argument and without any
 * allocation.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory -- code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc.  The scratch is a 16 MiB device
 * array in the library (one copy per GPU, held until the process ends; its
 * address is taken and the array zeroed on the first call on each device,
 * with that device current, and that first call waits for the fill, so it
 * must not be under stream capture); launches whose
 * tierkv_decode_workspace_bytes exceed 16 MiB fail with TIERKV_ERR_WORKSPACE.
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (different streams, or host threads) race.  Blocks skipped for an
 * out-of-range slot or state set the array's error word, which
 * tierkv_decode_noalloc_error_word reads.  Arguments and results otherwise
 * as tierkv_decode_attention; the stream must belong to the current
 * device. */
TIERKV_API int32_t tierkv_decode_attention_noalloc(
    const void* query, int32_t query_dtype, void* out, float* score_sums,
    const int32_t* block_table, const int32_t* block_states, const int32_t* block_lengths,
    int64_t table_stride, const int32_t* seq_num_blocks, int32_t num_blocks,
    const void* hot_k, const void* hot_v, int64_t hot_slots,
    const void* warm_k, const void* warm_v, int64_t warm_slots,
    const void* k_scale, const void* k_zero, const void* v_scale, const void* v_zero,
    int32_t warm_format, int32_t cold_mode,
    int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t block_size, int32_t head_dim,
    float scaling, int32_t splits_hint, void* stream);

/* The error word of the current device's allocation-free scratch (bit 1: a
 * resident block with an out-of-range slot was skipped; bit 2: a state that
 * is none of HOT/WARM/COLD), 0 before the first allocation-free launch on
 * the device; cleared when clear != 0.  Synchronises the device (a copy, no
 * allocation; not under stream capture).  Accessor of
 * tierkv_decode_attention_noalloc, likewise without a counterpart in the
 * reference. */
TIERKV_API int32_t tierkv_decode_noalloc_error_word(int32_t clear, int32_t* word);

/* Workspace bytes tierkv_decode_attention needs for this shape. */
TIERKV_API int64_t tierkv_decode_workspace_bytes(
    int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t num_blocks,
    int32_t block_size, int32_t head_dim, int32_t with_scores, int32_t splits_hint);

/* ---------------------------------------------------------------------- */
/* Demotion HOT -> WARM.  Replaces CompactTieredKVTensorPool.demote_to_warm
 * (tierkv_policy.py:1042-1068) / TieredKVTensorPool.demote_to_warm (329-361)
 * and quantize_fp16_to_int8 (21-36), batched: job i quantizes tiles
 * src_k/src_v[src_index[i]] (fp16 [kv_heads, block_size, head_dim], first
 * lengths[i] tokens) into warm slot dst_slot[i].  Jobs whose indices are out
 * of range are skipped (the Python layer validates them before launch).
 *   REF_U8: per (token, head) codes/scale/zero bit-exact with the
 *     reference's fp16 op sequence; tokens >= length are left untouched
 *     (pad_tail = 0, compact demote_to_warm) or zero-padded with scale 1 /
 *     zero 0 (pad_tail = 1, write_warm_block 989-995 / dense 350-356).
 *   ABSMAX_I8: scale = max|x| / 127 over the valid tokens of the (block,
 *     head) tile, codes rint(x / scale) clamped to [-127, 127]; tail codes 0.
 * table_pos  NULL, or int32 [n]: flat indices into block_table/block_states
 *   whose entries become (dst_slot[i], WARM) -- the _set_metadata rewrite
 *   (tierkv_policy.py:917-926); negative entries are skipped.
 */
TIERKV_API int32_t tierkv_demote_to_warm(
    const void* src_k, const void* src_v, int64_t src_tiles,
    const int32_t* src_index, const int32_t* dst_slot, const int32_t* lengths, int32_t n,
    void* warm_k, void* warm_v, int64_t warm_slots,
    void* k_scale, void* k_zero, void* v_scale, void* v_zero,
    int32_t warm_format, int32_t pad_tail,
    int32_t* block_table, int32_t* block_states, const int32_t* table_pos,
    int32_t num_kv_heads, int32_t block_size, int32_t head_dim, void* stream);

/* Promotion WARM -> HOT.  Replaces promote_to_hot (tierkv_policy.py:1087-1115,
 * 375-402) with dequantize_int8_to_fp16 (39-44): job i dequantizes the first
 * lengths[i] tokens of warm slot src_slot[i] into hot slot dst_slot[i]
 * (REF_U8: fp16 per-op rounding; ABSMAX_I8: fp16(fp32(q) * scale)).
 * table_pos as in tierkv_demote_to_warm, entries become (dst_slot[i], HOT). */
TIERKV_API int32_t tierkv_promote_to_hot(
    const void* warm_k, const void* warm_v, int64_t warm_slots,
    const void* k_scale, const void* k_zero, const void* v_scale, const void* v_zero,
    const int32_t* src_slot, const int32_t* dst_slot, const int32_t* lengths, int32_t n,
    void* hot_k, void* hot_v, int64_t hot_slots, int32_t warm_format,
    int32_t* block_table, int32_t* block_states, const int32_t* table_pos,
    int32_t num_kv_heads, int32_t block_size, int32_t head_dim, void* stream);

/* ---------------------------------------------------------------------- */
/* KV append into HOT slots.  Replaces the tensor copies of write_hot_tokens
 * (tierkv_policy.py:934-967; dense pool 238-267): job i copies tokens
 * [src_tok[i], src_tok[i] + count[i]) of sequence src_seq[i] of the fp16
 * sources src_k/src_v [src_seqs, kv_heads, src_tokens, head_dim] into HOT
 * slot dst_slot[i] at rows [dst_pos[i], dst_pos[i] + count[i]); with
 * zero_tail the slot's rows past the written range are zeroed, as the
 * reference does.  Jobs whose ranges fall outside their tensors are skipped. */
TIERKV_API int32_t tierkv_write_hot_tokens(
    const void* src_k, const void* src_v, int64_t src_seqs, int32_t src_tokens,
    const int32_t* src_seq, const int32_t* src_tok, const int32_t* count,
    const int32_t* dst_slot, const int32_t* dst_pos, int32_t n, int32_t zero_tail,
    void* hot_k, void* hot_v, int64_t hot_slots,
    int32_t num_kv_heads, int32_t block_size, int32_t head_dim, void* stream);

/* The same copy for at most 4 jobs given in HOST memory, jobs_host = int32
 * [n][5] = {src_seq, src_tok, count, dst_slot, dst_pos}: the jobs travel in
 * the kernel's arguments, so a decode step's single-token append needs no
 * host-to-device copy of its plan (write_hot_tokens, tierkv_policy.py:934-967,
 * as called once per layer and step by append_to_layer, 1768-1816). */
TIERKV_API int32_t tierkv_write_hot_tokens_inline(
    const void* src_k, const void* src_v, int64_t src_seqs, int32_t src_tokens, const int32_t* jobs_host, int32_t n,
    int32_t zero_tail, void* hot_k, void* hot_v, int64_t hot_slots,
    int32_t num_kv_heads, int32_t block_size, int32_t head_dim, void* stream);

/* Batched runtime (one layer of B sequences whose tables live on the device).
 * Free-slot stacks: int32 [capacity] arrays whose first `top` entries are free
 * slots; ctl is int32 [4] = {hot_top, warm_top, error bits, last append
 * applied (1) or refused (0)}.  Error bits: 1 no free HOT slot, 2 no free
 * WARM slot, 4 a table row is full, 8 a sequence's last block was not HOT. */

/* Append `tokens` new tokens per sequence from src_k/src_v [batch, kv_heads,
 * tokens, head_dim] fp16 at the end of each sequence's block list: the open
 * block first (the last block, when open_blocks[b] != 0), then new HOT blocks
 * popped from hot_free in sequence order (deterministic slot ids).
 * open_blocks [batch] is 1 while the last block was left partially filled by
 * an append; a prefill sets it to 0, since the reference starts decode
 * tokens in a new block (append_prefill_with_policy resets the open block,
 * tierkv_policy.py:1764-1766).  seq_num_blocks, open_blocks and the table
 * rows are updated on the device.  All-or-nothing when slots run out.  The
 * per-step part of append_to_layer (tierkv_policy.py:1768-1816) for a batch
 * of sequences, without host involvement.  blocks_hint: the block count the
 * caller expects every sequence to hold before the append (the lockstep
 * count a decode loop tracks), or 0; with it the last blocks' entries are
 * read together with the counts (one memory round trip less).  Results do
 * not depend on it. */
TIERKV_API int32_t tierkv_runtime_append(
    const void* src_k, const void* src_v, int32_t tokens,
    int32_t* block_table, int32_t* block_states, int32_t* block_lengths, int64_t table_stride,
    int32_t* seq_num_blocks, int32_t* open_blocks, int32_t batch, int32_t blocks_hint,
    void* hot_k, void* hot_v, int64_t hot_slots, int32_t* hot_free, int32_t* ctl,
    int32_t num_kv_heads, int32_t block_size, int32_t head_dim, void* stream);

/* tierkv_runtime_append with the decode step's rotary embedding fused in, for
 * fp16 models: K is rotated on its way into the pool, q is rotated into q_out
 * (contiguous fp16 [batch, num_heads, tokens, head_dim]), V is copied.  The
 * rotation is transformers' apply_rotary_pos_emb in its fp16 op order,
 * fp16(fp16(x * cos) + fp16(rotate_half(x) * sin)), so both are bit-identical
 * to it; it replaces the ~10 elementwise launches per layer that the HF hook
 * (modeling_llama.py:376-377) spends on the rotation.  q / k / v are fp16
 * [batch, heads, tokens, head_dim] with element strides (head_dim contiguous;
 * HF's projection views need no copy); cos / sin are fp16 [Bc, tokens,
 * head_dim] with strides (stride_b 0 broadcasts one row set over the batch).
 * head_dim a multiple of 16; every stride a multiple of 8 elements; every
 * pointer 16-byte aligned. */
TIERKV_API int32_t tierkv_runtime_append_rope(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_t, int32_t num_heads, void* q_out,
    const void* k, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_t,
    const void* v, int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_t,
    const void* cos, const void* sin, int64_t cs_stride_b, int64_t cs_stride_t, int32_t tokens,
    int32_t* block_table, int32_t* block_states, int32_t* block_lengths, int64_t table_stride,
    int32_t* seq_num_blocks, int32_t* open_blocks, int32_t batch, int32_t blocks_hint,
    void* hot_k, void* hot_v, int64_t hot_slots, int32_t* hot_free, int32_t* ctl,
    int32_t num_kv_heads, int32_t block_size, int32_t head_dim, void* stream);

/* One policy tick for one layer, entirely on the device: block scores from the
 * decode kernel's probability sums (block_scores_from_probability_sums,
 * tierkv_policy.py:1905-1912), stable-rank tier labels with reserved HOT
 * {0, n-1} and sticky COLD (enforce_budget mode 1 / enforce_tiered_budget
 * mode 2, 1391-1477), slot allocation (pops before pushes, in (sequence,
 * block) order) and the demote / promote data movement (sync_storage_states,
 * 1849-1867).  A migration that finds no free slot leaves its block as it is
 * and sets an error bit.  scratch: at least
 * tierkv_runtime_tick_scratch_bytes(...) bytes. */
TIERKV_API int32_t tierkv_runtime_tick(
    const float* score_sums, int64_t sums_stride, int32_t num_heads,
    int32_t* block_table, int32_t* block_states, int32_t* block_lengths, int64_t table_stride,
    const int32_t* seq_num_blocks, int32_t batch, int32_t hot_budget, int32_t warm_budget, int32_t mode,
    void* hot_k, void* hot_v, int64_t hot_slots, int32_t* hot_free,
    void* warm_k, void* warm_v, int64_t warm_slots, int32_t* warm_free,
    void* k_scale, void* k_zero, void* v_scale, void* v_zero, int32_t warm_format,
    int32_t* ctl, void* scratch, int64_t scratch_bytes, int32_t max_demotions, int32_t max_promotions,
    int32_t num_kv_heads, int32_t block_size, int32_t head_dim, void* stream);

TIERKV_API int64_t tierkv_runtime_tick_scratch_bytes(int32_t batch, int64_t table_stride,
                                                      int32_t max_demotions, int32_t max_promotions);

/* Prefill block scores without materialising the attention probabilities.
 * Replaces compute_block_scores on the prefill attention weights
 * (tierkv_policy.py:1380-1389 via modeling_llama.py:282-292), per sequence:
 *   mass[b, blk] = sum_{h, q} sum_{t in blk} p[b, h, q, t] / (H * T) / len(blk)
 * with p the causal softmax of scaling * q . k.  q [B, H, T, D] and k
 * [B, H_kv, T, D] are fp16 or bf16 with the given element strides (head_dim
 * contiguous, strides multiples of 8, 16-byte aligned); head_dim 64 or 128,
 * GQA group <= 8, block_size a multiple of 16, T <= 32768.  mass is fp32
 * [B, ceil(T / block_size)].  Two MFMA passes over K (log-sum-exp, then
 * block sums); deterministic (fixed reduction order).  workspace: at least
 * tierkv_prefill_block_mass_workspace_bytes(B, H_kv, T) bytes, no
 * initialisation needed. */
TIERKV_API int64_t tierkv_prefill_block_mass_workspace_bytes(int32_t batch, int32_t num_kv_heads, int32_t tokens);
TIERKV_API int32_t tierkv_prefill_block_mass(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_t,
    const void* k, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_t, int32_t dtype,
    float* mass, int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t tokens, int32_t head_dim,
    int32_t block_size, float scaling, void* workspace, int64_t workspace_bytes, void* stream);

/* Tier telemetry without a host sync: adds one layer's per-tier block and
 * token counts over sequences b < batch and blocks i < seq_num_blocks[b] into
 * counts int64[6] = {HOT, WARM, COLD blocks, HOT, WARM, COLD tokens} on the
 * device; the caller reads them back when it wants the numbers.  The counts
 * collect_memory_metrics derives from the tables (tierkv_policy.py:1193-1317,
 * 489-654) with one `.item()` sync per counter and layer. */
TIERKV_API int32_t tierkv_tier_counts(const int32_t* block_states, const int32_t* block_lengths,
                                      int64_t table_stride, const int32_t* seq_num_blocks, int32_t batch,
                                      int64_t* counts, void* stream);

/* Table writes planned on the host: dst[pairs[2i]] = pairs[2i + 1] for
 * i < n, positions distinct, out-of-range positions skipped; pairs is an
 * 8-byte-aligned int32 device array.  Replaces the per-entry device writes of
 * _set_metadata, set_block_entry, set_block_state and sync_gpu_block_tables
 * (tierkv_policy.py:917-926, 1019-1040, 1164-1174; dense pool 269-290,
 * 450-477), which the reference issues as one launch per table entry. */
TIERKV_API int32_t tierkv_scatter_i32(int32_t* dst, int64_t dst_len, const int32_t* pairs, int32_t n,
                                      void* stream);

/* The same writes for at most 16 pairs given in HOST memory (int32 [n][2]),
 * carried in the kernel's arguments: a decode step's table update (the open
 * block's length, a new block's entries) needs no host-to-device copy. */
TIERKV_API int32_t tierkv_scatter_i32_inline(int32_t* dst, int64_t dst_len, const int32_t* pairs_host, int32_t n,
                                             void* stream);

/* One decode step of a layer in one call: the token write of
 * tierkv_write_hot_tokens_inline (n_jobs 0..4), the table writes of
 * tierkv_scatter_i32_inline (n_pairs 0..16), then tierkv_decode_attention,
 * in stream order, each validated as its own entry point validates it; every
 * check runs before the first launch, so a call that returns an argument
 * error has queued nothing.  It
 * replaces the three calls the reference's decode forward makes per layer
 * and step (append_to_layer's token write, the table update it queues, and
 * tierkv_decode_attention: modeling_llama.py:419-456, tierkv_policy.py:
 * 1768-1816, 1869-1872), so that a host-bound caller pays one C call.  The
 * fields are those of the three entry points (8-byte fields first, so the
 * layout has no interior padding); tierkv_decode_step_size() returns
 * sizeof(TierkvDecodeStep) for bindings to check theirs against. */
typedef struct TierkvDecodeStep {
  const void* src_k;        /* token write: fp16 [src_seqs, kv_heads, src_tokens, head_dim] */
  const void* src_v;
  void* hot_k;              /* HOT pools: written by the token write, read by the decode */
  void* hot_v;
  int32_t* table_dst;       /* table writes: int32 [table_len] */
  const void* query;        /* decode: as tierkv_decode_attention */
  void* out;
  float* score_sums;
  const int32_t* block_table;
  const int32_t* block_states;
  const int32_t* block_lengths;
  const int32_t* seq_num_blocks;
  const void* warm_k;
  const void* warm_v;
  const void* k_scale;
  const void* k_zero;
  const void* v_scale;
  const void* v_zero;
  void* workspace;
  int64_t src_seqs;
  int64_t hot_slots;
  int64_t table_len;
  int64_t table_stride;
  int64_t warm_slots;
  int64_t workspace_bytes;
  int32_t src_tokens;
  int32_t n_jobs;
  int32_t zero_tail;
  int32_t n_pairs;
  int32_t query_dtype;
  int32_t num_blocks;
  int32_t warm_format;
  int32_t cold_mode;
  int32_t batch;
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t block_size;
  int32_t head_dim;
  float scaling;
  int32_t splits_hint;
  int32_t jobs[4][5];       /* {src_seq, src_tok, count, dst_slot, dst_pos} */
  int32_t pairs[16][2];     /* {table index, value} */
} TierkvDecodeStep;

TIERKV_API int32_t tierkv_decode_step(const TierkvDecodeStep* step, void* stream);
TIERKV_API int64_t tierkv_decode_step_size(void);

/* ---------------------------------------------------------------------- */
/* Block scores.  Per-block probability mass from softmax probabilities
 * probs fp32 [batch, num_heads, tokens] -> out fp32 [batch, tokens/block_size]:
 * sequential sum over heads, pairwise tree over the block's tokens, / heads,
 * / max(len, 1).  lengths NULL (full blocks) or int32 [batch, n_blocks].
 * The quantity of compute_block_scores (tierkv_policy.py:1380-1389) and
 * block_scores_from_probability_sums (1905-1912) for a batch of sequences. */
TIERKV_API int32_t tierkv_block_mass_from_probs(
    const float* probs, const int32_t* lengths, float* out,
    int32_t batch, int32_t num_heads, int32_t tokens, int32_t block_size, void* stream);

/* block_scores_from_probability_sums (tierkv_policy.py:1905-1912), batched:
 * score_sums fp32 [batch, num_heads, sums_stride], lengths int32
 * [batch, len_stride] -> out fp32 [batch, num_blocks]. */
TIERKV_API int32_t tierkv_block_scores_from_sums(
    const float* score_sums, int64_t sums_stride, const int32_t* lengths, int64_t len_stride,
    float* out, int32_t batch, int32_t num_heads, int32_t num_blocks, void* stream);

/* Tier labels.  TierKVPolicyEngine.enforce_tiered_budget (mode 2,
 * tierkv_policy.py:1434-1477) and enforce_budget (mode 1 with
 * demoted_state, 1391-1432) for a batch of sequences: reserved HOT
 * {0, n-1}, stable descending rank of the remaining scores, COLD sticky.
 * mode 0 (hot_only) copies cur_states.  scores fp32 [batch, n]; cur_states
 * and new_states int32 [batch, states_stride]. */
TIERKV_API int32_t tierkv_tier_labels(
    const float* scores, const int32_t* cur_states, int32_t* new_states, int64_t states_stride,
    int32_t batch, int32_t num_blocks, int32_t hot_budget, int32_t warm_budget,
    int32_t mode, int32_t demoted_state, void* stream);

/* ---------------------------------------------------------------------- */
/* BlockManager (host).  Replaces the pybind11 class of
 * csrc/block_manager.cpp:22-134 with identical allocation order and errors:
 * TIERKV_ERR_STATE carries the reference's message in tierkv_last_error(). */
typedef struct tierkv_block_manager tierkv_block_manager;

TIERKV_API int32_t tierkv_bm_create(int32_t total_blocks, tierkv_block_manager** out);   /* :24-34 */
TIERKV_API void tierkv_bm_destroy(tierkv_block_manager* bm);
TIERKV_API int32_t tierkv_bm_allocate_block(tierkv_block_manager* bm, int32_t seq_id, int32_t* physical_idx); /* :36-49 */
TIERKV_API int32_t tierkv_bm_free_sequence(tierkv_block_manager* bm, int32_t seq_id);   /* :51-62 */
TIERKV_API int32_t tierkv_bm_update_block_state(tierkv_block_manager* bm, int32_t seq_id,
                                     int32_t logical_id, int32_t state);     /* :64-77 */
/* Batched state write for logical ids [0, n) (a device policy tick's result);
 * same checks as update_block_state, applied to every entry before any write. */
TIERKV_API int32_t tierkv_bm_set_block_states(tierkv_block_manager* bm, int32_t seq_id,
                                   const int32_t* states, int32_t n);
TIERKV_API int32_t tierkv_bm_num_blocks(const tierkv_block_manager* bm, int32_t seq_id, int32_t* n);
/* Copy up to capacity entries; *n receives the full count (:79-105). */
TIERKV_API int32_t tierkv_bm_get_physical_indices(const tierkv_block_manager* bm, int32_t seq_id,
                                       int32_t* out, int32_t capacity, int32_t* n);
TIERKV_API int32_t tierkv_bm_get_states(const tierkv_block_manager* bm, int32_t seq_id,
                             int32_t* out, int32_t capacity, int32_t* n);
TIERKV_API int32_t tierkv_bm_num_free(const tierkv_block_manager* bm, int32_t* n);

#ifdef __cplusplus
}
#endif

#endif /* TIERKV_HIP_H */

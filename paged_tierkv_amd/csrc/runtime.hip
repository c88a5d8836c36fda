// Runtime kernels of the tiered KV cache on gfx950: KV append into HOT slots,
// device-side slot allocation and the device-side policy tick.
//
// Replaces, for the path's storage side:
//   * write_hot_tokens (tierkv_policy.py:934-967, dense 238-267): token
//     ranges copied into HOT slots, the rest of a written block zeroed;
//   * append_to_layer's per-step append (tierkv_policy.py:1768-1816) for a
//     batch of sequences, with new HOT blocks taken from a device free stack;
//   * one policy tick per layer: block_scores_from_probability_sums
//     (1905-1912), enforce_budget / enforce_tiered_budget (1391-1477) and
//     sync_storage_states (1849-1867) -- block scores, stable-rank labels,
//     slot allocation and the demote / promote data movement, with no host
//     round trip.
//
// Free stacks: int32 [capacity] arrays whose first `top` entries are free
// slots; the top counters live in a per-layer control word array
// ctl = {hot_top, warm_top, error bits, last append applied}.  Allocation pops from the top in
// a fixed order (sequence, then logical block), so slot ids are deterministic.

#include <algorithm>

#include "quantize.h"

namespace tierkv {

constexpr int RT = 1024;          // threads of the single-workgroup bookkeeping kernels
constexpr int CT = 256;           // threads per copy workgroup

// Error bits in ctl[2].
constexpr int ERR_HOT_EMPTY = 1;     // no free HOT slot for a new block or a promotion
constexpr int ERR_WARM_EMPTY = 2;    // no free WARM slot for a demotion
constexpr int ERR_TABLE_FULL = 4;    // a sequence exceeded its table row
constexpr int ERR_OPEN_STATE = 8;    // the last block of a sequence was not HOT

// Inclusive block-wide prefix sum of v over RT threads; returns the sum of
// all threads' values in *total.
__device__ int block_scan(int v, int* sh, int* total) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  if (lane == 63) sh[w] = x;
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int i = 0; i < RT / 64; ++i) {
      const int t = sh[i];
      sh[i] = run;
      run += t;
    }
    sh[RT / 64] = run;
  }
  __syncthreads();
  x += sh[w];
  *total = sh[RT / 64];
  __syncthreads();
  return x;
}

// ---------------------------------------------------------------------------
// write_hot_tokens: job i copies tokens [src_tok, src_tok + count) of sequence
// src_seq of src [S, kv_heads, T, D] into HOT slot dst_slot at positions
// [dst_pos, dst_pos + count); with zero_tail the block's positions past the
// written range are zeroed (tierkv_policy.py:955-960).
// ---------------------------------------------------------------------------
constexpr int INLINE_JOBS = 4;     // copy jobs carried by value in the kernel arguments
constexpr int INLINE_PAIRS = 16;   // table writes carried by value

struct CopyJobs {
  const __half* src[2];
  int64_t src_seqs;
  int32_t src_tokens;
  const int32_t* src_seq;
  const int32_t* src_tok;
  const int32_t* count;
  const int32_t* dst_slot;
  const int32_t* dst_pos;
  __half* hot[2];
  int64_t hot_slots;
  int32_t kv_heads, bs, D, zero_tail;
  // inl_n > 0: the jobs are inl[i] = {src_seq, src_tok, count, dst_slot,
  // dst_pos} (the pointers above are unused).
  int32_t inl_n;
  int32_t inl[INLINE_JOBS][5];
  // sc_n > 0: workgroup (0, 0, 0) also writes sc_dst[sc[i][0]] = sc[i][1]
  // (the table update of the same decode step, tierkv_decode_step).
  int32_t sc_n;
  int32_t* sc_dst;
  int64_t sc_len;
  int32_t sc[16][2];
};

__global__ __launch_bounds__(CT) void write_hot_kernel(CopyJobs c) {
  const int job = blockIdx.x;
  const int h = blockIdx.y;
  const int kv = blockIdx.z;
  if (c.sc_n > 0 && job == 0 && h == 0 && kv == 0 && int(threadIdx.x) < c.sc_n) {
    const int pos = c.sc[threadIdx.x][0], val = c.sc[threadIdx.x][1];
    if (pos >= 0 && pos < c.sc_len) c.sc_dst[pos] = val;
  }
  const bool inl = c.inl_n > 0;
  const int64_t sq = inl ? c.inl[job][0] : c.src_seq[job];
  const int64_t slot = inl ? c.inl[job][3] : c.dst_slot[job];
  const int t0 = inl ? c.inl[job][1] : c.src_tok[job];
  const int n = inl ? c.inl[job][2] : c.count[job];
  const int p0 = inl ? c.inl[job][4] : c.dst_pos[job];
  if (sq < 0 || sq >= c.src_seqs || slot < 0 || slot >= c.hot_slots) return;
  if (n < 0 || t0 < 0 || t0 + n > c.src_tokens || p0 < 0 || p0 + n > c.bs) return;
  const int D = c.D;
  const __half* src = c.src[kv] + ((sq * c.kv_heads + h) * int64_t(c.src_tokens) + t0) * D;
  __half* dst = c.hot[kv] + ((slot * c.kv_heads + h) * int64_t(c.bs) + p0) * D;
  const int end = c.zero_tail ? (c.bs - p0) * D : n * D;   // elements from dst
  const int copy = n * D;
  if ((D & 7) == 0 && ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15u) == 0) {
    const uint4* s4 = reinterpret_cast<const uint4*>(src);
    uint4* d4 = reinterpret_cast<uint4*>(dst);
    for (int e = threadIdx.x; e < end / 8; e += CT)
      d4[e] = (e < copy / 8) ? s4[e] : make_uint4(0u, 0u, 0u, 0u);
  } else {
    for (int e = threadIdx.x; e < end; e += CT) dst[e] = (e < copy) ? src[e] : __float2half(0.f);
  }
}

// ---------------------------------------------------------------------------
// Batched append: every sequence appends the same T tokens-count from
// src [B, kv_heads, T, D] at the end of its block list.  The open block is
// filled first: the last block, when open[b] says an earlier append left it
// partially filled (a prefill leaves no open block, as append_prefill_with_
// policy resets open_physical_idx, tierkv_policy.py:1764-1766).  Further
// tokens go to new HOT blocks popped from the free stack in sequence order,
// and open[b] records whether the new last block has room.  All-or-nothing:
// if the stack cannot cover every new block, nothing is appended and
// ERR_HOT_EMPTY is set.  One workgroup; meant for decode steps (a few tokens
// per sequence): B * 2 * kv_heads * T * D / 8 must stay below 2^31.
// ---------------------------------------------------------------------------
struct AppendParams {
  const __half* src[2];
  int64_t ss_b[2], ss_h[2], ss_t[2];   // element strides of the K / V sources [B, kv_heads, T, D]
  int32_t T;
  int32_t* table;
  int32_t* states;
  int32_t* lengths;
  int64_t stride;
  int32_t* nblocks;
  int32_t* open;
  __half* hot[2];
  int64_t hot_slots;
  int32_t* hot_free;
  int32_t* ctl;
  int32_t batch, kv_heads, bs, D;
  // Rotary embedding (rope != 0): K is rotated on its way into the pool and
  // q [B, heads, T, D] (strides qs_*) is rotated into q_out ([B, heads, T, D]
  // contiguous), with cos / sin [Bc, T, D] (cs_b = 0 broadcasts over the batch).
  int32_t rope;
  const __half* q;
  int64_t qs_b, qs_h, qs_t;
  __half* q_out;
  int32_t heads;
  const __half* cos;
  const __half* sin;
  int64_t cs_b, cs_t;
};

constexpr int APPEND_MAX_BATCH = 4096;   // sequences per append call (LDS bookkeeping)

// Eight consecutive elements [8c, 8c + 8) of a rotated row, in the fp16 op
// sequence of transformers' apply_rotary_pos_emb:
//   out = fp16(fp16(x * cos) + fp16(rotate_half(x) * sin)),
//   rotate_half(x)[d] = -x[d + D/2] (d < D/2), x[d - D/2] (d >= D/2).
// xv: the chunk, yv: its partner chunk in the other half, cv / sv: cos and
// sin of the chunk; lo: the chunk lies in the first half.
__device__ __forceinline__ uint4 rope8_vals(uint4 xv, uint4 yv, uint4 cv, uint4 sv, bool lo) {
  const __half* x = reinterpret_cast<const __half*>(&xv);
  const __half* y = reinterpret_cast<const __half*>(&yv);
  const __half* cs = reinterpret_cast<const __half*>(&cv);
  const __half* sn = reinterpret_cast<const __half*>(&sv);
  uint4 ov;
  __half* o = reinterpret_cast<__half*>(&ov);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float rot = lo ? -__half2float(y[i]) : __half2float(y[i]);
    const float p = __half2float(__float2half_rn(__half2float(x[i]) * __half2float(cs[i])));
    const float r = __half2float(__float2half_rn(rot * __half2float(sn[i])));
    o[i] = __float2half_rn(p + r);
  }
  return ov;
}

__device__ __forceinline__ uint4 rope8(const __half* row, const __half* cosr, const __half* sinr, int c, int D) {
  const int C2 = D / 16;                        // chunks per half row
  const bool lo = c < C2;
  return rope8_vals(*reinterpret_cast<const uint4*>(row + 8 * c),
                    *reinterpret_cast<const uint4*>(row + 8 * (lo ? c + C2 : c - C2)),
                    *reinterpret_cast<const uint4*>(cosr + 8 * c), *reinterpret_cast<const uint4*>(sinr + 8 * c), lo);
}

// Source row of an item.  The K / V choice is a select between the two
// parameter values: indexing the parameter arrays with a per-lane value
// would read them from the kernel-argument segment with vector loads, a
// dependent memory round trip per item.
template <typename P>
__device__ __forceinline__ const __half* kv_row(const P& a, int kv, int b, int h, int t) {
  const bool v = kv != 0;
  return (v ? a.src[1] : a.src[0]) + b * (v ? a.ss_b[1] : a.ss_b[0]) + h * (v ? a.ss_h[1] : a.ss_h[0]) +
         t * (v ? a.ss_t[1] : a.ss_t[0]);
}

// K / V item e of an append, e in [0, B * 2 * kv_heads * T * D / 8): eight
// elements [8c, 8c + 8) of token t of head h of K (kv 0) or V (kv 1) of
// sequence b.
struct KVItem {
  int b, kv, h, t, c;
};

__device__ __forceinline__ KVItem kv_item(int e, int H, int T, int C) {
  KVItem it;
  const int per_seq = 2 * H * T * C;
  it.b = e / per_seq;
  int r = e - it.b * per_seq;
  it.c = r % C;
  r /= C;
  it.t = r % T;
  r /= T;
  it.h = r % H;
  it.kv = r / H;
  return it;
}

// The loads of an item's 16 bytes, issued without using them: the chunk,
// and with the rotary embedding (ROPE) its partner chunk, cos and sin, for V
// items too (all in bounds; unused), so that no load sits behind a per-lane
// branch; kv_finish combines them (K rotated with ROPE).
struct KVRaw {
  uint4 x, y, c, s;
};
template <bool ROPE>
__device__ __forceinline__ KVRaw kv_raw(const AppendParams& a, const KVItem& it) {
  const uint4* row = reinterpret_cast<const uint4*>(kv_row(a, it.kv, it.b, it.h, it.t));
  KVRaw r;
  r.x = row[it.c];
  if constexpr (ROPE) {
    const int C2 = a.D / 16;
    r.y = row[it.c < C2 ? it.c + C2 : it.c - C2];
    r.c = reinterpret_cast<const uint4*>(a.cos + it.b * a.cs_b + it.t * a.cs_t)[it.c];
    r.s = reinterpret_cast<const uint4*>(a.sin + it.b * a.cs_b + it.t * a.cs_t)[it.c];
  }
  return r;
}
template <bool ROPE>
__device__ __forceinline__ uint4 kv_finish(const AppendParams& a, const KVItem& it, const KVRaw& r) {
  if constexpr (ROPE) return it.kv == 0 ? rope8_vals(r.x, r.y, r.c, r.s, it.c < a.D / 16) : r.x;
  return r.x;
}

constexpr int APPEND_NIT = APPEND_MAX_BATCH / RT;     // sequences per thread, at most

// Append bookkeeping (one workgroup): per sequence, the open block (flagged,
// last, HOT, not full) is filled first, then new HOT blocks popped from the
// free stack in sequence order; all-or-nothing over the batch.  Writes the
// table rows, block counts, open flags and the stack top, and ctl[3] = 1
// when the append was applied (0 when it was refused), which the copy
// kernel that follows reads.
// The leading arguments (read-only views of the counts, open flags and
// table rows, the row stride, the caller's block-count hint and the batch)
// are preloaded into scalar registers at wave launch, so the first table
// round trip needs no kernel-argument fetch; `hint` is the block count the
// caller expects every sequence to hold (0: none).  With it, the entries of
// the sequences' last blocks are loaded together with their counts, and
// only a sequence whose count differs takes another round trip.
__global__ __launch_bounds__(RT) void append_plan_kernel(const int32_t* r_nblocks, const int32_t* r_open,
                                                         const int32_t* r_lengths, const int32_t* r_states,
                                                         const int32_t* r_table, int32_t stride32, int32_t hint,
                                                         int32_t batch, AppendParams a) {
  __shared__ int sh[RT / 64 + 1];
  __shared__ int s_ok;
  const int tid = threadIdx.x;
  const int nit = (batch + RT - 1) / RT;
  int nb[APPEND_NIT], opn[APPEND_NIT], ln[APPEND_NIT], stt[APPEND_NIT], slot_open[APPEND_NIT];
#pragma unroll
  for (int it = 0; it < APPEND_NIT; ++it) {
    if (it < nit) {
      const int b = min(it * RT + tid, batch - 1);
      const int64_t o = int64_t(b) * stride32 + min(max(hint - 1, 0), stride32 - 1);
      nb[it] = r_nblocks[b];
      opn[it] = r_open[b];
      ln[it] = r_lengths[o];
      stt[it] = r_states[o];
      slot_open[it] = r_table[o];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  const int B = batch, bs = a.bs, T = a.T;
  const int top = a.ctl[0];
  if (tid == 0) s_ok = 1;
  int room[APPEND_NIT], len_open[APPEND_NIT], need[APPEND_NIT], excl[APPEND_NIT];
  // Sequences whose count is not the hint reload their last block's entries.
#pragma unroll
  for (int it = 0; it < APPEND_NIT; ++it) {
    if (it < nit && nb[it] != hint) {
      const int b = min(it * RT + tid, B - 1);
      const int64_t o = int64_t(b) * stride32 + min(max(nb[it] - 1, 0), stride32 - 1);
      ln[it] = r_lengths[o];
      stt[it] = r_states[o];
      slot_open[it] = r_table[o];
    }
  }
#pragma unroll
  for (int it = 0; it < APPEND_NIT; ++it) {
    room[it] = len_open[it] = need[it] = excl[it] = 0;
    const int b = it * RT + tid;
    if (it < nit && b < B) {
      if (nb[it] > 0 && nb[it] <= stride32 && opn[it] != 0) {
        const int len = min(max(ln[it], 0), bs);
        if (stt[it] != HOT) {
          if (len < bs) atomicOr(a.ctl + 2, ERR_OPEN_STATE);
        } else {
          len_open[it] = len;
          room[it] = bs - len;
        }
      }
      need[it] = T > room[it] ? (T - room[it] + bs - 1) / bs : 0;
    }
  }
  __syncthreads();
  int run = 0;
#pragma unroll
  for (int it = 0; it < APPEND_NIT; ++it) {
    if (it < nit) {
      const int b = it * RT + tid;
      if (b < B && (nb[it] < 0 || nb[it] + need[it] > stride32)) s_ok = 0;
      int tot;
      excl[it] = run + block_scan(need[it], sh, &tot) - need[it];
      run += tot;
    }
  }
  __syncthreads();
  if (!s_ok || run > top) {
    if (tid == 0) {
      atomicOr(a.ctl + 2, !s_ok ? ERR_TABLE_FULL : ERR_HOT_EMPTY);
      a.ctl[3] = 0;
    }
    return;
  }
  // Table entries; new blocks pop the stack in sequence order.
#pragma unroll
  for (int it = 0; it < APPEND_NIT; ++it) {
    const int b = it * RT + tid;
    if (it < nit && b < B) {
      const int take_open = min(room[it], T);
      if (take_open > 0) a.lengths[int64_t(b) * a.stride + nb[it] - 1] = len_open[it] + take_open;
      for (int j = 0; j < need[it]; ++j) {
        const int64_t o = int64_t(b) * a.stride + nb[it] + j;
        a.table[o] = a.hot_free[top - 1 - (excl[it] + j)];
        a.states[o] = HOT;
        a.lengths[o] = min(T - take_open - j * bs, bs);
      }
      a.nblocks[b] = nb[it] + need[it];
      const int last_len = need[it] > 0 ? min(T - take_open - (need[it] - 1) * bs, bs) : len_open[it] + take_open;
      a.open[b] = last_len < bs ? 1 : 0;
    }
  }
  if (tid == 0) {
    a.ctl[0] = top - run;
    a.ctl[3] = 1;
  }
}

// Append copies (after append_plan_kernel): one 16-byte K / V item per
// thread, rotated for K with the rotary embedding (ROPE), stored into the
// HOT pool; workgroups past the K / V items rotate the query rows (ROPE).
// The destination comes from the rows the plan wrote: an append fills its
// sequence contiguously (the open block's free rows, then new blocks from
// row 0), so its T tokens are the last T valid rows of the row list, and
// token t lies T - 1 - t rows before the end.  Nothing is stored when the
// plan refused the append (ctl[3] == 0).  The source loads, the status and
// the block count are issued together; the last block's entries follow.
// Rows past a block's length are not cleared: pools start zeroed and only
// ever hold finite fp16 values, and every consumer masks rows by length.
template <bool ROPE>
__global__ __launch_bounds__(CT) void append_copy_kernel(AppendParams a, int32_t kv_groups) {
  const int B = a.batch, bs = a.bs, T = a.T;
  const int D = a.D, C = D / 8, H = a.kv_heads;
  if (ROPE && int(blockIdx.x) >= kv_groups) {
    const int per_seq = a.heads * T * C;
    const int total = B * per_seq;
    const int nq = int(gridDim.x) - kv_groups;
    for (int e = (int(blockIdx.x) - kv_groups) * CT + int(threadIdx.x); e < total; e += nq * CT) {
      const int b = e / per_seq;
      int r = e - b * per_seq;
      const int c = r % C;
      r /= C;
      const int t = r % T;
      const int qh = r / T;
      const __half* row = a.q + b * a.qs_b + qh * a.qs_h + t * a.qs_t;
      const __half* cr = a.cos + b * a.cs_b + t * a.cs_t;
      const __half* sr = a.sin + b * a.cs_b + t * a.cs_t;
      reinterpret_cast<uint4*>(a.q_out + ((int64_t(b) * a.heads + qh) * T + t) * D)[c] = rope8(row, cr, sr, c, D);
    }
    return;
  }
  const int total_kv = B * 2 * H * T * C;
  const int e = int(blockIdx.x) * CT + int(threadIdx.x);
  if (e >= total_kv) return;
  const KVItem it = kv_item(e, H, T, C);
  const KVRaw raw = kv_raw<ROPE>(a, it);
  const int applied = a.ctl[3];
  int blk = a.nblocks[it.b] - 1;
  __builtin_amdgcn_sched_barrier(0);
  if (!applied || blk < 0) return;
  // Walk back over the row list to the token's block.
  int r = T - 1 - it.t;
  int len = min(max(a.lengths[int64_t(it.b) * a.stride + blk], 0), bs);
  while (r >= len && blk > 0) {
    r -= len;
    --blk;
    len = min(max(a.lengths[int64_t(it.b) * a.stride + blk], 0), bs);
  }
  if (r >= len) return;
  const int64_t slot = a.table[int64_t(it.b) * a.stride + blk];
  if (slot < 0 || slot >= a.hot_slots) return;
  __half* pool = it.kv ? a.hot[1] : a.hot[0];
  reinterpret_cast<uint4*>(pool + ((slot * H + it.h) * int64_t(bs) + (len - 1 - r)) * D)[it.c] =
      kv_finish<ROPE>(a, it, raw);
}

// ---------------------------------------------------------------------------
// Policy tick for one layer of a batch of sequences.
// ---------------------------------------------------------------------------
struct TickParams {
  const float* score_sums;   // [B, heads, sums_stride]
  int64_t sums_stride;
  int32_t heads;
  int32_t* table;
  int32_t* states;
  int32_t* lengths;
  int64_t stride;
  const int32_t* nblocks;
  int32_t batch;
  int32_t hot_budget, warm_budget, mode;   // mode 1: demoted blocks WARM, 2: WARM budget then COLD
  int32_t* hot_free;
  int32_t* warm_free;
  int32_t* ctl;
  float* scores;      // [B, stride] scratch: block scores
  int32_t* labels;    // [B, stride] scratch: desired states
  int32_t* dem;       // [3][max_dem] demotion jobs (src hot slot, dst warm slot, length)
  int32_t* pro;       // [3][max_pro] promotion jobs (src warm slot, dst hot slot, length)
  int32_t* counts;    // [2] demotions, promotions
  int32_t max_dem, max_pro;
};

// Block scores and tier labels, one workgroup per sequence.
//   Scores: the mean over heads of the per-block probability sums, divided
//   by max(length, 1) (block_scores_from_probability_sums), with the same
//   operations in the same order as tierkv_block_scores_from_sums; a
//   thread's head values are loaded together (TICK_HEADS per round) before
//   they are summed in head order.
//   Labels: reserved HOT {0, n-1}; candidates ranked by score descending
//   with ties to the lower index (Python's stable sort, as the 64-bit label
//   keys order them); COLD never leaves COLD.  The row's scores are kept in
//   LDS (rows up to TICK_LDS_BLOCKS; longer rows read them back from the
//   scratch), and every thread ranks its candidates against the whole row.
constexpr int LT = 512;
constexpr int TICK_HEADS = 32;
constexpr int TICK_LDS_BLOCKS = 8192;
__global__ __launch_bounds__(LT) void tick_label_kernel(TickParams t) {
  extern __shared__ float s_sc[];   // [n] scores when n <= TICK_LDS_BLOCKS
  const int tid = threadIdx.x;
  const int b = blockIdx.x;
  const int n = min(max(t.nblocks[b], 0), int(t.stride));
  const int64_t ob = int64_t(b) * t.stride;
  const bool in_lds = n <= TICK_LDS_BLOCKS;
  for (int i0 = 0; i0 < n; i0 += LT) {
    const int i = min(i0 + tid, n - 1);
    const float* p = t.score_sums + int64_t(b) * t.heads * t.sums_stride + i;
    const int len = max(t.lengths[ob + i], 1);
    float acc = 0.f;
    for (int h0 = 0; h0 < t.heads; h0 += TICK_HEADS) {
      float v[TICK_HEADS];
#pragma unroll
      for (int k = 0; k < TICK_HEADS; ++k) v[k] = p[int64_t(min(h0 + k, t.heads - 1)) * t.sums_stride];
#pragma unroll
      for (int k = 0; k < TICK_HEADS; ++k)
        if (h0 + k < t.heads) acc += v[k];
    }
    const float sc = __fdiv_rn(__fdiv_rn(acc, float(t.heads)), float(len));
    if (i0 + tid < n) {
      t.scores[ob + i] = sc;
      if (in_lds) s_sc[i] = sc;
    }
  }
  __syncthreads();
  auto score = [&](int j) -> float { return in_lds ? s_sc[j] : t.scores[ob + j]; };
  const int extra_hot = max(t.hot_budget - 2, 0);
  const uint64_t k_first = n > 2 ? label_key(score(0), 0) : 0;
  const uint64_t k_last = n > 2 ? label_key(score(n - 1), n - 1) : 0;
  for (int i = tid; i < n; i += LT) {
    const bool cand = n > 2 && i > 0 && i < n - 1;
    const uint64_t ki = cand ? label_key(score(i), i) : ~uint64_t(0);
    int rank = 0;
    for (int j = 0; j < n; ++j) rank += label_key(score(j), j) > ki ? 1 : 0;
    // blocks 0 and n - 1 are reserved, not candidates
    rank -= (k_first > ki ? 1 : 0) + (k_last > ki ? 1 : 0);
    const int cur = t.states[ob + i];
    int want;
    if (!cand) {
      want = HOT;
    } else if (rank < extra_hot) {
      want = HOT;
    } else if (t.mode == 2) {
      want = (rank < extra_hot + max(t.warm_budget, 0)) ? WARM : COLD;
    } else {
      want = WARM;
    }
    if (cur == COLD) want = COLD;
    t.labels[ob + i] = want;
  }
}

// Slot allocation and table rewrite of a tick (one workgroup), after
// tick_label_kernel.  Slots freed by the tick are reused within it, in the
// order the data movement allows (demotions run before promotions):
//   1. the WARM slots of WARM -> COLD blocks are pushed on the WARM stack;
//   2. demotions (HOT -> WARM) pop the WARM stack;
//   3. the HOT slots of demoted and HOT -> COLD blocks are pushed on the
//      HOT stack;
//   4. promotions (WARM -> HOT) pop the HOT stack;
//   5. the WARM slots of promoted blocks are pushed on the WARM stack.
// Every step goes in (sequence, block) order, so slot ids are
// deterministic.  A demotion never lands in a slot a promotion still has to
// read (promoted slots are pushed last) and a promotion may land in a slot a
// demotion reads (the demotion kernel runs first).  So the pools need the
// budgets, not twice the HOT budget: between ticks a sequence holds at most
// its HOT budget plus the blocks appended since, and at most its WARM budget
// plus its promotions during a tick.  A migration that gets no slot is left
// undone.  Three passes over the (sequence, block) cells, one block scan of
// two 0/1 flags each (16 bits per flag: a scan's prefix is at most RT); with
// at most TICK_KEPT * RT cells each thread loads its cells once.
constexpr int TICK_KEPT = 4;
struct TickCell {
  int cur, want, slot, len;
};
__global__ __launch_bounds__(RT) void tick_plan_kernel(TickParams t) {
  __shared__ int sh[RT / 64 + 1];
  const int tid = threadIdx.x;
  const int B = t.batch;
  const int hot_top = t.ctl[0];
  const int warm_top = t.ctl[1];
  // Cells past the last sequence's count are never live: N bounds them.
  const int64_t N = int64_t(B - 1) * t.stride + min(max(t.nblocks[B - 1], 0), int(t.stride));
  auto load_cell = [&](int64_t e) -> TickCell {
    const int64_t ec = min(e, max(N - 1, int64_t(0)));
    const int b = int(ec / t.stride);
    const int i = int(ec - int64_t(b) * t.stride);
    const int n = t.nblocks[b];
    TickCell c{t.states[ec], t.labels[ec], t.table[ec], t.lengths[ec]};
    if (!(e < N && i < min(max(n, 0), int(t.stride)))) c.cur = c.want = COLD;
    return c;
  };
  const bool kept = N <= int64_t(TICK_KEPT) * RT;
  TickCell cell[TICK_KEPT];
  if (kept) {
#pragma unroll
    for (int k = 0; k < TICK_KEPT; ++k) cell[k] = load_cell(int64_t(k) * RT + tid);
  }
  // One sweep over the cells with a pass body f(e, cell).
  auto sweep = [&](auto&& f) {
    if (kept) {
#pragma unroll
      for (int k = 0; k < TICK_KEPT; ++k)
        if (int64_t(k) * RT < N) f(int64_t(k) * RT + tid, cell[k]);
    } else {
      for (int64_t e0 = 0; e0 < N; e0 += RT) f(e0 + tid, load_cell(e0 + tid));
    }
    __syncthreads();
  };
  auto is_dem = [](const TickCell& c) { return (c.cur == HOT && c.want == WARM) ? 1 : 0; };
  auto is_pro = [](const TickCell& c) { return (c.cur == WARM && c.want == HOT) ? 1 : 0; };

  // Pass A: push the WARM slots of WARM -> COLD blocks; count demotions and
  // promotions.
  __shared__ int s_np;
  if (tid == 0) s_np = 0;
  __syncthreads();
  int ev_run = 0, d_run = 0;
  sweep([&](int64_t, const TickCell& c) {
    const int ew = (c.cur == WARM && c.want == COLD) ? 1 : 0;
    int tot;
    const int inc = block_scan(ew | (is_dem(c) << 16), sh, &tot);
    if (ew) t.warm_free[warm_top + ev_run + (inc & 0xffff) - 1] = c.slot;
    if (is_pro(c)) atomicAdd(&s_np, 1);
    ev_run += tot & 0xffff;
    d_run += tot >> 16;
  });
  const int np_total = s_np;
  const int wtop1 = warm_top + ev_run;                      // WARM stack after step 1
  const int ndem = min(min(d_run, wtop1), t.max_dem);

  // Pass B: demotion jobs (the first ndem demotions pop the WARM stack) and
  // the pushes of freed HOT slots (demoted or HOT -> COLD blocks): a cell's
  // push position counts the demoted and the HOT -> COLD cells before it.
  int dk_run = 0, eh_run = 0;
  sweep([&](int64_t, const TickCell& c) {
    const int d = is_dem(c);
    const int eh = (c.cur == HOT && c.want == COLD) ? 1 : 0;
    int tot;
    const int inc = block_scan(d | (eh << 16), sh, &tot);
    const int dk = (inc & 0xffff) - d + dk_run;
    const int ehk = (inc >> 16) - eh + eh_run;
    if (d) {
      if (dk < ndem) {
        t.dem[dk] = c.slot;
        t.dem[t.max_dem + dk] = t.warm_free[wtop1 - 1 - dk];
        t.dem[2 * t.max_dem + dk] = c.len;
      } else {
        atomicOr(t.ctl + 2, ERR_WARM_EMPTY);
      }
    }
    if ((d && dk < ndem) || eh) t.hot_free[hot_top + min(dk, ndem) + ehk] = c.slot;
    dk_run += tot & 0xffff;
    eh_run += tot >> 16;
  });
  const int htop1 = hot_top + ndem + eh_run;                // HOT stack after step 3
  const int npro = min(min(np_total, htop1), t.max_pro);

  // Pass C: promotion jobs (the first npro promotions pop the HOT stack),
  // the pushes of promoted blocks' WARM slots, and the table rewrite.
  int pk_run = 0, dk2_run = 0;
  sweep([&](int64_t e, const TickCell& c) {
    const int d = is_dem(c);
    const int p = is_pro(c);
    int tot;
    const int inc = block_scan(p | (d << 16), sh, &tot);
    const int pk = (inc & 0xffff) - p + pk_run;
    const int dk = (inc >> 16) - d + dk2_run;
    const bool d_ok = d && dk < ndem;
    const bool p_ok = p && pk < npro;
    if (p && !p_ok) atomicOr(t.ctl + 2, ERR_HOT_EMPTY);
    if (p_ok) {
      const int hs = t.hot_free[htop1 - 1 - pk];
      t.pro[pk] = c.slot;
      t.pro[t.max_pro + pk] = hs;
      t.pro[2 * t.max_pro + pk] = c.len;
      t.warm_free[wtop1 - ndem + pk] = c.slot;
      t.table[e] = hs;
      t.states[e] = HOT;
    } else if (d_ok) {
      t.table[e] = t.dem[t.max_dem + dk];
      t.states[e] = WARM;
    } else if (c.want == COLD && c.cur != COLD) {
      t.table[e] = -1;
      t.states[e] = COLD;
    }
    pk_run += tot & 0xffff;
    dk2_run += tot >> 16;
  });
  if (tid == 0) {
    t.ctl[0] = htop1 - npro;
    t.ctl[1] = wtop1 - ndem + npro;
    t.counts[0] = ndem;
    t.counts[1] = npro;
  }
}

// ---------------------------------------------------------------------------
// Host-planned table writes: dst[pairs[2i]] = pairs[2i + 1].  The host
// coalesces its writes per position, so positions are distinct and the
// launch order of the pairs does not matter.
// ---------------------------------------------------------------------------
struct InlinePairs {
  int32_t n;
  int32_t v[2 * INLINE_PAIRS];
};

// The same writes with the pairs carried by value (at most INLINE_PAIRS).
__global__ __launch_bounds__(64) void scatter_i32_inline_kernel(int32_t* dst, int64_t len, InlinePairs p) {
  const int i = threadIdx.x;
  if (i >= p.n) return;
  const int pos = p.v[2 * i], val = p.v[2 * i + 1];
  if (pos >= 0 && pos < len) dst[pos] = val;
}

__global__ __launch_bounds__(CT) void scatter_i32_kernel(int32_t* dst, int64_t len, const int32_t* pairs, int n) {
  const int i = blockIdx.x * CT + threadIdx.x;
  if (i >= n) return;
  const int2 pv = reinterpret_cast<const int2*>(pairs)[i];
  if (pv.x >= 0 && pv.x < len) dst[pv.x] = pv.y;
}

// ---------------------------------------------------------------------------
// Tier telemetry: per-tier block and token counts of one layer, added into
// counts[6] = {HOT, WARM, COLD blocks, HOT, WARM, COLD tokens} (int64).  One
// workgroup; LDS partial sums, one global add per counter.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(CT) void tier_counts_kernel(const int32_t* states, const int32_t* lengths,
                                                         int64_t stride, const int32_t* nblocks, int batch,
                                                         int max_blocks, unsigned long long* counts) {
  __shared__ unsigned long long s_cnt[6];
  if (threadIdx.x < 6) s_cnt[threadIdx.x] = 0ull;
  __syncthreads();
  unsigned long long c[6] = {0ull, 0ull, 0ull, 0ull, 0ull, 0ull};
  for (int b = 0; b < batch; ++b) {
    const int n = min(max(nblocks[b], 0), max_blocks);
    for (int i = threadIdx.x; i < n; i += CT) {
      const int64_t o = int64_t(b) * stride + i;
      const int st = states[o];
      if (st < 0 || st > 2) continue;
      c[st] += 1ull;
      c[3 + st] += static_cast<unsigned long long>(max(lengths[o], 0));
    }
  }
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    unsigned long long v = c[k];
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
    if ((threadIdx.x & 63) == 0 && v) atomicAdd(&s_cnt[k], v);
  }
  __syncthreads();
  if (threadIdx.x < 6) atomicAdd(&counts[threadIdx.x], s_cnt[threadIdx.x]);
}

}  // namespace tierkv

using namespace tierkv;

extern "C" int32_t tierkv_tier_counts(const int32_t* block_states, const int32_t* block_lengths,
                                      int64_t table_stride, const int32_t* seq_num_blocks, int32_t batch,
                                      int64_t* counts, void* stream) {
  clear_error();
  if (!block_states || !block_lengths || !seq_num_blocks || !counts) return fail(TIERKV_ERR_INVALID, "null pointer");
  if (batch <= 0 || table_stride <= 0 || table_stride > 0x7fffffff) return fail(TIERKV_ERR_INVALID, "bad table geometry");
  hipLaunchKernelGGL(tier_counts_kernel, dim3(1), dim3(CT), 0, reinterpret_cast<hipStream_t>(stream), block_states,
                     block_lengths, table_stride, seq_num_blocks, batch, int(table_stride),
                     reinterpret_cast<unsigned long long*>(counts));
  return check_launch("tier_counts_kernel");
}

extern "C" int32_t tierkv_scatter_i32(int32_t* dst, int64_t dst_len, const int32_t* pairs, int32_t n,
                                      void* stream) {
  clear_error();
  if (n < 0) return fail(TIERKV_ERR_INVALID, "negative pair count");
  if (n == 0) return TIERKV_OK;
  if (!dst || !pairs) return fail(TIERKV_ERR_INVALID, "null pointer");
  if ((reinterpret_cast<uintptr_t>(pairs) & 7u) != 0) return fail(TIERKV_ERR_INVALID, "pairs must be 8-byte aligned");
  if (dst_len > 0x7fffffff) return fail(TIERKV_ERR_UNSUPPORTED, "scatter target above 2^31 entries");
  hipLaunchKernelGGL(scatter_i32_kernel, dim3((n + CT - 1) / CT), dim3(CT), 0,
                     reinterpret_cast<hipStream_t>(stream), dst, dst_len, pairs, n);
  return check_launch("scatter_i32_kernel");
}

extern "C" int32_t tierkv_scatter_i32_inline(int32_t* dst, int64_t dst_len, const int32_t* pairs_host, int32_t n,
                                             void* stream) {
  clear_error();
  if (n < 0 || n > INLINE_PAIRS) return fail(TIERKV_ERR_INVALID, "inline scatter takes 0..16 pairs");
  if (n == 0) return TIERKV_OK;
  if (!dst || !pairs_host) return fail(TIERKV_ERR_INVALID, "null pointer");
  if (dst_len > 0x7fffffff) return fail(TIERKV_ERR_UNSUPPORTED, "scatter target above 2^31 entries");
  InlinePairs p{};
  p.n = n;
  for (int i = 0; i < 2 * n; ++i) p.v[i] = pairs_host[i];
  hipLaunchKernelGGL(scatter_i32_inline_kernel, dim3(1), dim3(64), 0, reinterpret_cast<hipStream_t>(stream), dst,
                     dst_len, p);
  return check_launch("scatter_i32_inline_kernel");
}

static int32_t check_write_geometry(const void* src_k, const void* src_v, const void* hot_k, const void* hot_v,
                                    int32_t src_tokens, int32_t num_kv_heads, int32_t block_size, int32_t head_dim);

extern "C" int32_t tierkv_decode_step(const TierkvDecodeStep* s, void* stream) {
  clear_error();
  if (!s) return fail(TIERKV_ERR_INVALID, "null pointer");
  if (s->n_jobs < 0 || s->n_jobs > INLINE_JOBS) return fail(TIERKV_ERR_INVALID, "a step carries 0..4 write jobs");
  if (s->n_pairs < 0 || s->n_pairs > INLINE_PAIRS) return fail(TIERKV_ERR_INVALID, "a step carries 0..16 table writes");
  // The decode launch's arguments are checked before the token write goes
  // out, so a refused step leaves the device as it was.
  {
    const int32_t rc = decode_check_args(
        s->query, s->query_dtype, s->out, s->score_sums, s->block_table, s->block_states, s->block_lengths,
        s->table_stride, s->num_blocks, s->hot_k, s->hot_v, s->hot_slots, s->warm_k, s->warm_v, s->warm_slots,
        s->k_scale, s->k_zero, s->v_scale, s->v_zero, s->warm_format, s->cold_mode, s->batch, s->num_heads,
        s->num_kv_heads, s->block_size, s->head_dim, s->splits_hint, s->workspace, s->workspace_bytes);
    if (rc != TIERKV_OK) return rc;
  }
  if (s->n_jobs > 0) {
    // The token write and the table writes in one launch: workgroup (0, 0, 0)
    // of the write kernel also applies the pairs.
    int32_t rc = check_write_geometry(s->src_k, s->src_v, s->hot_k, s->hot_v, s->src_tokens, s->num_kv_heads,
                                      s->block_size, s->head_dim);
    if (rc != TIERKV_OK) return rc;
    if (s->n_pairs > 0 && !s->table_dst) return fail(TIERKV_ERR_INVALID, "null pointer");
    if (s->table_len > 0x7fffffff) return fail(TIERKV_ERR_UNSUPPORTED, "scatter target above 2^31 entries");
    CopyJobs c{};
    c.src[0] = reinterpret_cast<const __half*>(s->src_k);
    c.src[1] = reinterpret_cast<const __half*>(s->src_v);
    c.src_seqs = s->src_seqs;
    c.src_tokens = s->src_tokens;
    c.hot[0] = reinterpret_cast<__half*>(s->hot_k);
    c.hot[1] = reinterpret_cast<__half*>(s->hot_v);
    c.hot_slots = s->hot_slots;
    c.kv_heads = s->num_kv_heads;
    c.bs = s->block_size;
    c.D = s->head_dim;
    c.zero_tail = s->zero_tail;
    c.inl_n = s->n_jobs;
    for (int i = 0; i < s->n_jobs; ++i)
      for (int f = 0; f < 5; ++f) c.inl[i][f] = s->jobs[i][f];
    c.sc_n = s->n_pairs;
    c.sc_dst = s->table_dst;
    c.sc_len = s->table_len;
    for (int i = 0; i < s->n_pairs; ++i) {
      c.sc[i][0] = s->pairs[i][0];
      c.sc[i][1] = s->pairs[i][1];
    }
    hipLaunchKernelGGL(write_hot_kernel, dim3(s->n_jobs, s->num_kv_heads, 2), dim3(CT), 0,
                       reinterpret_cast<hipStream_t>(stream), c);
    rc = check_launch("write_hot_kernel");
    if (rc != TIERKV_OK) return rc;
  } else if (s->n_pairs > 0) {
    const int32_t rc = tierkv_scatter_i32_inline(s->table_dst, s->table_len, &s->pairs[0][0], s->n_pairs, stream);
    if (rc != TIERKV_OK) return rc;
  }
  return tierkv_decode_attention(s->query, s->query_dtype, s->out, s->score_sums, s->block_table, s->block_states,
                                 s->block_lengths, s->table_stride, s->seq_num_blocks, s->num_blocks, s->hot_k,
                                 s->hot_v, s->hot_slots, s->warm_k, s->warm_v, s->warm_slots, s->k_scale, s->k_zero,
                                 s->v_scale, s->v_zero, s->warm_format, s->cold_mode, s->batch, s->num_heads,
                                 s->num_kv_heads, s->block_size, s->head_dim, s->scaling, s->splits_hint,
                                 s->workspace, s->workspace_bytes, stream);
}

extern "C" int64_t tierkv_decode_step_size(void) { return int64_t(sizeof(TierkvDecodeStep)); }

static int32_t check_write_geometry(const void* src_k, const void* src_v, const void* hot_k, const void* hot_v,
                                    int32_t src_tokens, int32_t num_kv_heads, int32_t block_size, int32_t head_dim) {
  if (!src_k || !src_v || !hot_k || !hot_v) return fail(TIERKV_ERR_INVALID, "null pointer");
  if (num_kv_heads <= 0 || block_size <= 0 || block_size > 64 || head_dim <= 0 || head_dim > 256 || src_tokens <= 0)
    return fail(TIERKV_ERR_UNSUPPORTED, "block_size must be in [1, 64] and head_dim in [1, 256]");
  if (num_kv_heads > 65535) return fail(TIERKV_ERR_UNSUPPORTED, "too many kv heads");
  return TIERKV_OK;
}

extern "C" int32_t tierkv_write_hot_tokens_inline(
    const void* src_k, const void* src_v, int64_t src_seqs, int32_t src_tokens, const int32_t* jobs_host, int32_t n,
    int32_t zero_tail, void* hot_k, void* hot_v, int64_t hot_slots,
    int32_t num_kv_heads, int32_t block_size, int32_t head_dim, void* stream) {
  clear_error();
  if (n < 0 || n > INLINE_JOBS) return fail(TIERKV_ERR_INVALID, "inline write takes 0..4 jobs");
  if (n == 0) return TIERKV_OK;
  if (!jobs_host) return fail(TIERKV_ERR_INVALID, "null pointer");
  const int32_t rc = check_write_geometry(src_k, src_v, hot_k, hot_v, src_tokens, num_kv_heads, block_size, head_dim);
  if (rc != TIERKV_OK) return rc;
  CopyJobs c{};
  c.src[0] = reinterpret_cast<const __half*>(src_k);
  c.src[1] = reinterpret_cast<const __half*>(src_v);
  c.src_seqs = src_seqs;
  c.src_tokens = src_tokens;
  c.hot[0] = reinterpret_cast<__half*>(hot_k);
  c.hot[1] = reinterpret_cast<__half*>(hot_v);
  c.hot_slots = hot_slots;
  c.kv_heads = num_kv_heads;
  c.bs = block_size;
  c.D = head_dim;
  c.zero_tail = zero_tail;
  c.inl_n = n;
  for (int i = 0; i < n; ++i)
    for (int f = 0; f < 5; ++f) c.inl[i][f] = jobs_host[5 * i + f];
  hipLaunchKernelGGL(write_hot_kernel, dim3(n, num_kv_heads, 2), dim3(CT), 0,
                     reinterpret_cast<hipStream_t>(stream), c);
  return check_launch("write_hot_kernel");
}

extern "C" int32_t tierkv_write_hot_tokens(
    const void* src_k, const void* src_v, int64_t src_seqs, int32_t src_tokens,
    const int32_t* src_seq, const int32_t* src_tok, const int32_t* count,
    const int32_t* dst_slot, const int32_t* dst_pos, int32_t n, int32_t zero_tail,
    void* hot_k, void* hot_v, int64_t hot_slots,
    int32_t num_kv_heads, int32_t block_size, int32_t head_dim, void* stream) {
  clear_error();
  if (n < 0) return fail(TIERKV_ERR_INVALID, "negative job count");
  if (n == 0) return TIERKV_OK;
  if (!src_k || !src_v || !src_seq || !src_tok || !count || !dst_slot || !dst_pos || !hot_k || !hot_v)
    return fail(TIERKV_ERR_INVALID, "null pointer");
  if (num_kv_heads <= 0 || block_size <= 0 || block_size > 64 || head_dim <= 0 || head_dim > 256 || src_tokens <= 0)
    return fail(TIERKV_ERR_UNSUPPORTED, "block_size must be in [1, 64] and head_dim in [1, 256]");
  if (n > 65535 * 64) return fail(TIERKV_ERR_UNSUPPORTED, "too many copy jobs in one call");
  CopyJobs c{};
  c.src[0] = reinterpret_cast<const __half*>(src_k);
  c.src[1] = reinterpret_cast<const __half*>(src_v);
  c.src_seqs = src_seqs;
  c.src_tokens = src_tokens;
  c.src_seq = src_seq;
  c.src_tok = src_tok;
  c.count = count;
  c.dst_slot = dst_slot;
  c.dst_pos = dst_pos;
  c.hot[0] = reinterpret_cast<__half*>(hot_k);
  c.hot[1] = reinterpret_cast<__half*>(hot_v);
  c.hot_slots = hot_slots;
  c.kv_heads = num_kv_heads;
  c.bs = block_size;
  c.D = head_dim;
  c.zero_tail = zero_tail;
  hipLaunchKernelGGL(write_hot_kernel, dim3(n, num_kv_heads, 2), dim3(CT), 0,
                     reinterpret_cast<hipStream_t>(stream), c);
  return check_launch("write_hot_kernel");
}

// The two launches of an append: bookkeeping (one workgroup), then one
// copy thread per 16-byte K / V item (and q_groups query-rotation
// workgroups with ROPE).
template <bool ROPE>
static int32_t launch_append(const AppendParams& a, const int32_t* nblocks, const int32_t* open,
                             const int32_t* lengths, const int32_t* states, const int32_t* table, int32_t stride32,
                             int32_t hint, int32_t batch, int q_groups, hipStream_t stream) {
  hipLaunchKernelGGL(append_plan_kernel, dim3(1), dim3(RT), 0, stream, nblocks, open, lengths, states, table, stride32,
                     hint, batch, a);
  const int32_t rc = check_launch("append_plan_kernel");
  if (rc != TIERKV_OK) return rc;
  const int64_t total_kv = int64_t(batch) * 2 * a.kv_heads * a.T * (a.D / 8);
  const int kv_groups = static_cast<int>((total_kv + CT - 1) / CT);
  hipLaunchKernelGGL(append_copy_kernel<ROPE>, dim3(kv_groups + q_groups), dim3(CT), 0, stream, a, kv_groups);
  return check_launch("append_copy_kernel");
}

extern "C" int32_t tierkv_runtime_append(
    const void* src_k, const void* src_v, int32_t tokens,
    int32_t* block_table, int32_t* block_states, int32_t* block_lengths, int64_t table_stride,
    int32_t* seq_num_blocks, int32_t* open_blocks, int32_t batch, int32_t blocks_hint,
    void* hot_k, void* hot_v, int64_t hot_slots, int32_t* hot_free, int32_t* ctl,
    int32_t num_kv_heads, int32_t block_size, int32_t head_dim, void* stream) {
  clear_error();
  if (!src_k || !src_v || !block_table || !block_states || !block_lengths || !seq_num_blocks || !open_blocks ||
      !hot_k || !hot_v || !hot_free || !ctl)
    return fail(TIERKV_ERR_INVALID, "null pointer");
  if (batch <= 0 || tokens <= 0 || table_stride <= 0) return fail(TIERKV_ERR_INVALID, "empty append");
  if (table_stride > 0x7fffffff) return fail(TIERKV_ERR_UNSUPPORTED, "table rows too long");
  if (batch > APPEND_MAX_BATCH) return fail(TIERKV_ERR_UNSUPPORTED, "append supports at most 4096 sequences per call");
  if (int64_t(batch) * 2 * num_kv_heads * tokens * (head_dim / 8) >= (int64_t(1) << 31))
    return fail(TIERKV_ERR_UNSUPPORTED, "append too large for one call");
  if (num_kv_heads <= 0 || block_size <= 0 || block_size > 64 || head_dim <= 0 || head_dim > 256 ||
      head_dim % 8 != 0)
    return fail(TIERKV_ERR_UNSUPPORTED, "block_size must be in [1, 64] and head_dim a multiple of 8 up to 256");
  if (!aligned16(src_k) || !aligned16(src_v) || !aligned16(hot_k) || !aligned16(hot_v))
    return fail(TIERKV_ERR_INVALID, "KV sources and HOT pools must be 16-byte aligned");
  AppendParams a{};
  a.src[0] = reinterpret_cast<const __half*>(src_k);
  a.src[1] = reinterpret_cast<const __half*>(src_v);
  for (int kv = 0; kv < 2; ++kv) {
    a.ss_t[kv] = head_dim;
    a.ss_h[kv] = int64_t(tokens) * head_dim;
    a.ss_b[kv] = int64_t(num_kv_heads) * tokens * head_dim;
  }
  a.T = tokens;
  a.table = block_table;
  a.states = block_states;
  a.lengths = block_lengths;
  a.stride = table_stride;
  a.nblocks = seq_num_blocks;
  a.open = open_blocks;
  a.hot[0] = reinterpret_cast<__half*>(hot_k);
  a.hot[1] = reinterpret_cast<__half*>(hot_v);
  a.hot_slots = hot_slots;
  a.hot_free = hot_free;
  a.ctl = ctl;
  a.batch = batch;
  a.kv_heads = num_kv_heads;
  a.bs = block_size;
  a.D = head_dim;
  return launch_append<false>(a, seq_num_blocks, open_blocks, block_lengths, block_states, block_table,
                              int32_t(table_stride), blocks_hint, batch, 0, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int32_t tierkv_runtime_append_rope(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_t, int32_t num_heads, void* q_out,
    const void* k, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_t,
    const void* v, int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_t,
    const void* cos, const void* sin, int64_t cs_stride_b, int64_t cs_stride_t, int32_t tokens,
    int32_t* block_table, int32_t* block_states, int32_t* block_lengths, int64_t table_stride,
    int32_t* seq_num_blocks, int32_t* open_blocks, int32_t batch, int32_t blocks_hint,
    void* hot_k, void* hot_v, int64_t hot_slots, int32_t* hot_free, int32_t* ctl,
    int32_t num_kv_heads, int32_t block_size, int32_t head_dim, void* stream) {
  clear_error();
  if (!q || !q_out || !k || !v || !cos || !sin || !block_table || !block_states || !block_lengths ||
      !seq_num_blocks || !open_blocks || !hot_k || !hot_v || !hot_free || !ctl)
    return fail(TIERKV_ERR_INVALID, "null pointer");
  if (batch <= 0 || tokens <= 0 || table_stride <= 0 || num_heads <= 0) return fail(TIERKV_ERR_INVALID, "empty append");
  if (table_stride > 0x7fffffff) return fail(TIERKV_ERR_UNSUPPORTED, "table rows too long");
  if (batch > APPEND_MAX_BATCH) return fail(TIERKV_ERR_UNSUPPORTED, "append supports at most 4096 sequences per call");
  if (int64_t(batch) * (2 * num_kv_heads + num_heads) * tokens * (head_dim / 8) >= (int64_t(1) << 31))
    return fail(TIERKV_ERR_UNSUPPORTED, "append too large for one call");
  if (num_kv_heads <= 0 || block_size <= 0 || block_size > 64 || head_dim <= 0 || head_dim > 256 ||
      head_dim % 16 != 0)
    return fail(TIERKV_ERR_UNSUPPORTED, "block_size must be in [1, 64] and head_dim a multiple of 16 up to 256");
  const int64_t strides[11] = {q_stride_b, q_stride_h, q_stride_t, k_stride_b, k_stride_h, k_stride_t,
                               v_stride_b, v_stride_h, v_stride_t, cs_stride_b, cs_stride_t};
  for (int64_t st : strides)
    if (st < 0 || st % 8 != 0) return fail(TIERKV_ERR_INVALID, "strides must be non-negative multiples of 8 elements");
  const void* ptrs[7] = {q, q_out, k, v, cos, sin, hot_k};
  for (const void* ptr : ptrs)
    if (!aligned16(ptr)) return fail(TIERKV_ERR_INVALID, "q, k, v, cos, sin, q_out and pools must be 16-byte aligned");
  if (!aligned16(hot_v)) return fail(TIERKV_ERR_INVALID, "HOT pools must be 16-byte aligned");
  AppendParams a{};
  a.src[0] = reinterpret_cast<const __half*>(k);
  a.src[1] = reinterpret_cast<const __half*>(v);
  a.ss_b[0] = k_stride_b;
  a.ss_h[0] = k_stride_h;
  a.ss_t[0] = k_stride_t;
  a.ss_b[1] = v_stride_b;
  a.ss_h[1] = v_stride_h;
  a.ss_t[1] = v_stride_t;
  a.T = tokens;
  a.table = block_table;
  a.states = block_states;
  a.lengths = block_lengths;
  a.stride = table_stride;
  a.nblocks = seq_num_blocks;
  a.open = open_blocks;
  a.hot[0] = reinterpret_cast<__half*>(hot_k);
  a.hot[1] = reinterpret_cast<__half*>(hot_v);
  a.hot_slots = hot_slots;
  a.hot_free = hot_free;
  a.ctl = ctl;
  a.batch = batch;
  a.kv_heads = num_kv_heads;
  a.bs = block_size;
  a.D = head_dim;
  a.rope = 1;
  a.q = reinterpret_cast<const __half*>(q);
  a.qs_b = q_stride_b;
  a.qs_h = q_stride_h;
  a.qs_t = q_stride_t;
  a.q_out = reinterpret_cast<__half*>(q_out);
  a.heads = num_heads;
  a.cos = reinterpret_cast<const __half*>(cos);
  a.sin = reinterpret_cast<const __half*>(sin);
  a.cs_b = cs_stride_b;
  a.cs_t = cs_stride_t;
  // Copy workgroups past the K / V items rotate the query rows.
  const int64_t q_items = int64_t(batch) * num_heads * tokens * (head_dim / 8);
  const int q_groups = static_cast<int>(std::min<int64_t>((q_items + CT - 1) / CT, 1024));
  return launch_append<true>(a, seq_num_blocks, open_blocks, block_lengths, block_states, block_table,
                             int32_t(table_stride), blocks_hint, batch, q_groups, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int32_t tierkv_runtime_tick(
    const float* score_sums, int64_t sums_stride, int32_t num_heads,
    int32_t* block_table, int32_t* block_states, int32_t* block_lengths, int64_t table_stride,
    const int32_t* seq_num_blocks, int32_t batch, int32_t hot_budget, int32_t warm_budget, int32_t mode,
    void* hot_k, void* hot_v, int64_t hot_slots, int32_t* hot_free,
    void* warm_k, void* warm_v, int64_t warm_slots, int32_t* warm_free,
    void* k_scale, void* k_zero, void* v_scale, void* v_zero, int32_t warm_format,
    int32_t* ctl, void* scratch, int64_t scratch_bytes, int32_t max_demotions, int32_t max_promotions,
    int32_t num_kv_heads, int32_t block_size, int32_t head_dim, void* stream_) {
  clear_error();
  if (!score_sums || !block_table || !block_states || !block_lengths || !seq_num_blocks || !hot_k || !hot_v ||
      !hot_free || !warm_k || !warm_v || !warm_free || !k_scale || !v_scale || !ctl || !scratch)
    return fail(TIERKV_ERR_INVALID, "null pointer");
  if (mode != 1 && mode != 2) return fail(TIERKV_ERR_INVALID, "tick mode must be 1 (hot_warm) or 2 (hot_warm_cold)");
  if (warm_format == TIERKV_WARM_REF_U8 && (!k_zero || !v_zero))
    return fail(TIERKV_ERR_INVALID, "reference format needs zero-point pools");
  if (batch <= 0 || num_heads <= 0 || table_stride <= 0 || sums_stride < table_stride)
    return fail(TIERKV_ERR_INVALID, "bad tick geometry");
  if (max_demotions < 0 || max_promotions < 0 || max_demotions > 65535 * 64 || max_promotions > 65535 * 64)
    return fail(TIERKV_ERR_INVALID, "bad job bounds");
  if (num_kv_heads <= 0 || block_size <= 0 || block_size > 64 || head_dim <= 0 || head_dim > 256)
    return fail(TIERKV_ERR_UNSUPPORTED, "block_size must be in [1, 64] and head_dim in [1, 256]");
  const int64_t cells = int64_t(batch) * table_stride;
  const int64_t need = cells * 8 + (int64_t(max_demotions) + max_promotions) * 12 + 16;
  if (scratch_bytes < need) return fail(TIERKV_ERR_WORKSPACE, "tick scratch too small");
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  char* s = reinterpret_cast<char*>(scratch);
  TickParams t{};
  t.score_sums = score_sums;
  t.sums_stride = sums_stride;
  t.heads = num_heads;
  t.table = block_table;
  t.states = block_states;
  t.lengths = block_lengths;
  t.stride = table_stride;
  t.nblocks = seq_num_blocks;
  t.batch = batch;
  t.hot_budget = hot_budget;
  t.warm_budget = warm_budget;
  t.mode = mode;
  t.hot_free = hot_free;
  t.warm_free = warm_free;
  t.ctl = ctl;
  t.scores = reinterpret_cast<float*>(s);
  t.labels = reinterpret_cast<int32_t*>(s + cells * 4);
  t.dem = reinterpret_cast<int32_t*>(s + cells * 8);
  t.pro = t.dem + 3 * int64_t(max_demotions);
  t.counts = t.pro + 3 * int64_t(max_promotions);
  t.max_dem = max_demotions;
  t.max_pro = max_promotions;
  const size_t lds = table_stride <= TICK_LDS_BLOCKS ? size_t(table_stride) * sizeof(float) : 0;
  hipLaunchKernelGGL(tick_label_kernel, dim3(batch), dim3(LT), lds, stream, t);
  int32_t rc = check_launch("tick_label_kernel");
  if (rc != TIERKV_OK) return rc;
  hipLaunchKernelGGL(tick_plan_kernel, dim3(1), dim3(RT), 0, stream, t);
  rc = check_launch("tick_plan_kernel");
  if (rc != TIERKV_OK) return rc;

  QuantJobs q{};
  q.src[0] = reinterpret_cast<const __half*>(hot_k);
  q.src[1] = reinterpret_cast<const __half*>(hot_v);
  q.src_tiles = hot_slots;
  q.src_index = t.dem;
  q.dst_slot = t.dem + max_demotions;
  q.lengths = t.dem + 2 * int64_t(max_demotions);
  q.warm[0] = warm_k;
  q.warm[1] = warm_v;
  q.warm_slots = warm_slots;
  q.scale[0] = k_scale;
  q.scale[1] = v_scale;
  q.zero[0] = k_zero;
  q.zero[1] = v_zero;
  q.kv_heads = num_kv_heads;
  q.bs = block_size;
  q.D = head_dim;
  q.pad_tail = 0;
  q.n_dev = t.counts;
  rc = launch_demote(q, max_demotions, warm_format, stream);
  if (rc != TIERKV_OK) return rc;

  DequantJobs d{};
  d.warm[0] = warm_k;
  d.warm[1] = warm_v;
  d.warm_slots = warm_slots;
  d.scale[0] = k_scale;
  d.scale[1] = v_scale;
  d.zero[0] = k_zero;
  d.zero[1] = v_zero;
  d.src_slot = t.pro;
  d.dst_slot = t.pro + max_promotions;
  d.lengths = t.pro + 2 * int64_t(max_promotions);
  d.hot[0] = reinterpret_cast<__half*>(hot_k);
  d.hot[1] = reinterpret_cast<__half*>(hot_v);
  d.hot_slots = hot_slots;
  d.kv_heads = num_kv_heads;
  d.bs = block_size;
  d.D = head_dim;
  d.warm_format = warm_format;
  d.n_dev = t.counts + 1;
  return launch_promote(d, max_promotions, stream);
}

extern "C" int64_t tierkv_runtime_tick_scratch_bytes(int32_t batch, int64_t table_stride, int32_t max_demotions,
                                                      int32_t max_promotions) {
  if (batch <= 0 || table_stride <= 0 || max_demotions < 0 || max_promotions < 0) return -1;
  return int64_t(batch) * table_stride * 8 + (int64_t(max_demotions) + max_promotions) * 12 + 16;
}

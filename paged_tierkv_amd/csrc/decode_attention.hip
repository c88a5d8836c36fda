// Tiered paged decode attention for gfx950 (CDNA4).
//
// Replaces _tierkv_decode_attention_kernel (tierkv_triton.py:45-145) and the
// split/reduce pair (147-264) behind tierkv_decode_attention
// (tierkv_triton.py:272-465).
//
// Fast path (block_size 16, head_dim 64 or 128, GQA group <= 16), one kernel
// (a second one finalises the score sums of split launches):
//   * workgroup = (sequence, kv head, split), 8 waves (4 when the GQA group
//     exceeds 8); the whole GQA group is served by one pass over each K/V
//     byte; unsplit launches of a batch that is a multiple of 8 place each
//     sequence's kv heads on one XCD;
//   * every workgroup scans its sequence's table row and keeps its share of
//     the resident blocks, HOT and WARM ranked separately: a contiguous range
//     of each tier's ranks when the row fits one pass of the build, the ranks
//     congruent to its split otherwise; COLD blocks cost no bytes;
//   * one wave handles one 16-token block (tile) at a time with MFMA
//     16x16x16 f16:  S^T = K Q^T  (A = K rows as loaded, B = Q^T), then
//     O^T += V^T P^T  (B = P^T is exactly S^T's accumulator layout); tiles
//     are handed to waves from LDS counters as they free up, or in fixed
//     interleaved shares (TIERKV_DECODE_DETERMINISTIC);
//   * WARM codes become fp16 by a byte permute under the exponent of 1024
//     (int8 absmax codes + 1152, uint8 reference codes + 1024, exactly); the
//     constant offset (and the reference format's zero points) is removed
//     once per head from the logits and by one more MFMA from the output,
//     and the scales are folded into the logits and into P;
//   * the next tile is prefetched into a second register buffer (ping-pong),
//     the tier branch is wave-uniform;
//   * online softmax in base 2 whose running maximum is re-based only when a
//     logit exceeds it by more than LAZY_T (P stays <= 2^LAZY_T);
//   * waves merge in LDS; when a sequence is split over several workgroups
//     the last one to finish (an atomic counter per (sequence, kv head))
//     merges the partials (log-sum-exp combine, tierkv_triton.py:231-264);
//   * score launches stage each visited block's (max, sum) per head and
//     reduce every head's row along a fixed tree, so the per-block
//     probability sums (tierkv_triton.py:121-145) are the same bits whatever
//     the tile order and split count: unsplit launches whose statistics fit
//     the workgroup's LDS finalise in the workgroup, the others (split
//     launches, longer rows) in finalize_scores_kernel.
// Generic path (any block_size <= 64, head_dim <= 256, any group): one wave
// per (sequence, q head), the reference kernel's structure.

#include "tierkv_common.h"

#include <algorithm>
#include <type_traits>
#include <cfloat>
#include <cmath>
#include <mutex>

namespace tierkv {

constexpr int FBS = 16;            // tokens per block on the fast path
constexpr int MAX_LIST = 512;      // resident blocks per workgroup (LDS list)
constexpr int MAX_WAVES = 8;
constexpr int PRE_CHUNKS = 4;      // table-row chunks loaded together by the list build
constexpr int MERGE_UNROLL = 8;    // split partials loaded together by the merge
constexpr int MAX_LDS_STAGE = 48 * 1024;   // bytes of per-block score statistics kept in LDS
// Where a score launch stages each block's (max, sum) per head:
//   STAGE_LDS_BLOCK LDS [G][num_blocks] by logical block (unsplit launches),
//                   finalised by the workgroup itself;
//   STAGE_LDS_LIST  LDS [G][MAX_LIST] by list position, copied to the
//                   workspace [B][H][num_blocks] at the end of the workgroup
//                   (split launches);
//   STAGE_GLOBAL    the workspace, written per tile (rows too long for LDS).
// The workspace stages are finalised by finalize_scores_kernel, launched
// after the decode kernel: one workgroup per (sequence, q head) row spreads
// that work over the chip, where a unit's last workgroup would read every
// staged pair of the unit and write its whole score rows from one CU.
constexpr int STAGE_GLOBAL = 0;
constexpr int STAGE_LDS_BLOCK = 1;
constexpr int STAGE_LDS_LIST = 2;
constexpr int MAX_SPLIT_UNITS = 1 << 16;   // units per launch when a unit is split
constexpr float PBOOST = 64.f;     // P is scaled by 2^6 before its fp16 cast
constexpr float LAZY_T = 8.f;      // log2 headroom of the running maximum
constexpr float FOLD_MAX = 2.f;    // WARM V scales above this are applied to V
constexpr uint32_t FOLD_MAX_F16 = 0x4000u;   // FOLD_MAX as an fp16 bit pattern
constexpr float LOG2E = 1.4426950408889634f;
constexpr float BIAS_I8 = 1152.f;  // fp16 value of an int8 code c is 1152 + c
constexpr float BIAS_U8 = 1024.f;  // fp16 value of a uint8 code u is 1024 + u
constexpr uint32_t BIAS_I8_F16X2 = 0x64806480u;   // two fp16 1152s

struct DecodeParams {
  const void* q;
  void* out;
  const int32_t* table;
  const int32_t* states;
  const int32_t* lengths;
  int64_t table_stride;
  const int32_t* seq_nblocks;
  int32_t num_blocks;
  const __half* hot_k;
  const __half* hot_v;
  int64_t hot_slots;
  const void* warm_k;
  const void* warm_v;
  int64_t warm_slots;
  const void* k_scale;
  const void* k_zero;
  const void* v_scale;
  const void* v_zero;
  int32_t batch, num_heads, kv_heads, block_size, head_dim, groups;
  float scale_log2;   // scaling * log2(e)
  float scaling;
  int32_t splits;
  uint32_t split_magic;   // ceil(2^32 / splits) when num_blocks * splits < 2^32, else 0
  int32_t lds_stage;      // where score statistics are staged (STAGE_* below)
  int32_t deterministic;  // host only: fixed tile shares per wave (TIERKV_DECODE_DETERMINISTIC)
  float* ws_acc;      // [units][splits][G][D]
  float* ws_ml;       // [units][splits][G][2]
  float* ws_stage;    // [B][H][num_blocks][2]  per-block (max, sum) (split score launches)
  uint32_t* ws_cnt;   // [MAX_SPLIT_UNITS] split arrival counters, zero between launches
  int32_t* ws_err;
  float* score_sums;  // [B][H][table_stride] or null
};

// Arrival of a split workgroup on its unit's counter; returns the arrivals
// before this one.  The counters live in a region of the workspace that no
// other data shares and are zero between launches: the last arrival of each
// unit resets its counter.  The caller has waited for its partial's stores.
__device__ __forceinline__ uint32_t arrive(uint32_t* c) {
  return __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ int seq_blocks(const DecodeParams& p, int b) {
  int nb = p.num_blocks;
  if (p.seq_nblocks) nb = min(max(p.seq_nblocks[b], 0), p.num_blocks);
  return nb;
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Device-coherent (agent scope) relaxed stores and loads: the store is
// written through to the level shared by all XCDs, the load does not hit a
// stale copy.  Workgroups of one split exchange partials and per-block
// statistics with them; ordering comes from waiting for the stores to
// complete before the arrival counter is incremented.
__device__ __forceinline__ void store_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_dev(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Workgroup barrier that orders LDS accesses only.  __syncthreads() also
// waits for the wave's outstanding global stores (on gfx9 they count in the
// same vector-memory counter as loads), which the score finalisation would
// otherwise pay for right after the output stores.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// --------------------------------------------------------------------------
// Fast path
// --------------------------------------------------------------------------

// Tiles in registers.  Lane (n = lane & 15, g = lane >> 4) holds
//   k: token n; HOT: dims 32i + 8g .. +7 of load i, WARM: dims 64i + 16g
//      .. +15 of load i (each load instruction covers whole 64-byte row
//      segments);
//   v: tokens 4g + j (j = 0..3), dims n*D/16 .. +D/16 (row j at v[j*RW]);
// HOT tiles as fp16 pairs, WARM tiles as 8-bit codes plus metadata
// (absmax: s_k, s_v, two 4-byte loads).  The reference format's four
// per-token rows (k scale, k zero, v scale, v zero of the (block, head), 32
// bytes each) are one load instruction: lane 4q + a of each quad fetches
// row a's 8 bytes for tokens 4g .. 4g+3, and warm_meta spreads them over
// the quad with DPP broadcasts when the tile is processed (four separate
// loads: C3 40.7 us; one: 39.9 us).  The two tiers have their own
// registers: each tile loop is straight-line code for one tier.
template <int D>
struct HotTile {
  static constexpr int RW = D / 32;   // dwords per V row
  uint32_t k[D / 8];
  uint32_t v[D / 8];
};

template <int D, int WF>
struct WarmTile {
  static constexpr int RW = D / 64;
  static constexpr int NR = 2;                                        // metadata dwords as loaded
  static constexpr int NM = (WF == TIERKV_WARM_ABSMAX_I8) ? 2 : 8;   // after warm_meta
  uint32_t k[D / 16];
  uint32_t v[D / 16];
  uint32_t mr[NR];
};

// Value of lane 4 * (lane / 4) + A (DPP quad_perm [A, A, A, A]).
template <int A>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
  return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), A * 0x55, 0xf, 0xf, false));
}

// The tile's metadata in every lane: absmax m[0] = s_k, m[1] = s_v;
// reference format m[0..7] = fp16 pairs of the k scale, k zero, v scale and
// v zero of tokens 4g .. 4g+3.
template <int D, int WF>
__device__ __forceinline__ void warm_meta(const WarmTile<D, WF>& t, uint32_t* m) {
  if constexpr (WF == TIERKV_WARM_ABSMAX_I8) {
    m[0] = t.mr[0];
    m[1] = t.mr[1];
  } else {
    m[0] = quad_bcast<0>(t.mr[0]); m[1] = quad_bcast<0>(t.mr[1]);
    m[2] = quad_bcast<1>(t.mr[0]); m[3] = quad_bcast<1>(t.mr[1]);
    m[4] = quad_bcast<2>(t.mr[0]); m[5] = quad_bcast<2>(t.mr[1]);
    m[6] = quad_bcast<3>(t.mr[0]); m[7] = quad_bcast<3>(t.mr[1]);
  }
}

// Tile loads go through buffer resources built per tile in scalar registers
// (base = the tile's first byte, num_records = its size).  A dead load (a
// pipeline step past the end of the list) gets num_records = 0: every lane is
// out of range, the hardware returns zeros without a memory access, and the
// load retires quickly, so a wave leaving its loop does not wait for a memory
// round trip before its registers can be reused.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
constexpr int RSRC_WORD3 = 0x00020000;   // gfx9 buffer descriptor: raw 32-bit dwords
// Cache policy of the tile loads: non-temporal.  Every tile byte is read once
// per launch; the streaming hint keeps the tiles from displacing other lines
// and measurably raises gather bandwidth on gfx950.
#ifndef TIERKV_TILE_CPOL
#define TIERKV_TILE_CPOL 2
#endif
constexpr int TILE_CPOL = TIERKV_TILE_CPOL;
// Tiles in flight per wave (register pipeline depth) in the HOT and WARM
// loops.
#ifndef TIERKV_NBH
#define TIERKV_NBH 2
#endif
#ifndef TIERKV_NBW
#define TIERKV_NBW 2
#endif

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, RSRC_WORD3);
}

// Where a WARM tile's metadata comes from, set up once per workgroup:
// absmax, one buffer resource per scale array (a tile's scale is an offset
// into it, and a dead pipeline step's offset is the array's size, which
// reads nothing); the reference format, this lane's row array (the piece it
// loads for every tile).  Resources per tile would hold four more scalar
// registers per tile in flight, which the long-row kernels do not have.
template <int WF>
struct WarmMeta {
  __amdgpu_buffer_rsrc_t ks, vs;   // absmax
  uint32_t bytes;                  // absmax: size of each scale array
  const char* row;                 // reference format
};

template <int WF>
__device__ __forceinline__ WarmMeta<WF> warm_meta_setup(const DecodeParams& p, int lane) {
  WarmMeta<WF> m{};
  if constexpr (WF == TIERKV_WARM_ABSMAX_I8) {
    // The host keeps warm_slots * kv_heads * 4 below 2^32.
    m.bytes = uint32_t(p.warm_slots * p.kv_heads * 4);
    m.ks = tile_rsrc(p.k_scale, m.bytes);
    m.vs = tile_rsrc(p.v_scale, m.bytes);
  } else {
    const int a = lane & 3;
    m.row = static_cast<const char*>(a == 0 ? p.k_scale : a == 1 ? p.k_zero : a == 2 ? p.v_scale : p.v_zero);
  }
  return m;
}

template <int D>
__device__ __forceinline__ void load_hot(const DecodeParams& p, int kvh, int slot, int lane, HotTile<D>& t,
                                         bool live) {
  const int n = lane & 15;
  const int g = lane >> 4;
  constexpr uint32_t TILE = FBS * D * 2;
  const int64_t tile0 = (int64_t(slot) * p.kv_heads + kvh) * FBS;   // first token row of the tile
  const auto rk = tile_rsrc(p.hot_k + tile0 * D, live ? TILE : 0u);
  const auto rv = tile_rsrc(p.hot_v + tile0 * D, live ? TILE : 0u);
  // Instruction i reads bytes [64i, 64i + 64) of every row (whole lines);
  // lane g's 16 bytes are dims 32i + 8g .. +7 (the query's HOT permutation).
  const int ko = n * (D * 2) + 16 * g;
#pragma unroll
  for (int i = 0; i < D / 32; ++i) {
    const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rk, ko + 64 * i, 0, TILE_CPOL);
    t.k[4 * i + 0] = x.x; t.k[4 * i + 1] = x.y; t.k[4 * i + 2] = x.z; t.k[4 * i + 3] = x.w;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int vo = ((4 * g + j) * D + n * (D / 16)) * 2;
    if constexpr (D == 128) {
      const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rv, vo, 0, TILE_CPOL);
      t.v[4 * j + 0] = x.x; t.v[4 * j + 1] = x.y; t.v[4 * j + 2] = x.z; t.v[4 * j + 3] = x.w;
    } else {
      const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(rv, vo, 0, TILE_CPOL);
      t.v[2 * j + 0] = x.x; t.v[2 * j + 1] = x.y;
    }
  }
}

template <int D, int WF>
__device__ __forceinline__ void load_warm(const DecodeParams& p, int kvh, int slot, int lane, const WarmMeta<WF>& wm,
                                          WarmTile<D, WF>& t, bool live) {
  const int n = lane & 15;
  const int g = lane >> 4;
  constexpr uint32_t TILE = FBS * D;
  const int64_t tile0 = (int64_t(slot) * p.kv_heads + kvh) * FBS;
  const auto rk = tile_rsrc(reinterpret_cast<const uint8_t*>(p.warm_k) + tile0 * D, live ? TILE : 0u);
  const auto rv = tile_rsrc(reinterpret_cast<const uint8_t*>(p.warm_v) + tile0 * D, live ? TILE : 0u);
  // Instruction i reads bytes [64i, 64i + 64) of every row (whole 64-byte
  // segments, as for HOT K); lane g's 16 bytes are dims 64i + 16g .. +15.
  const int ko = n * D + 16 * g;
#pragma unroll
  for (int i = 0; i < D / 64; ++i) {
    const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rk, ko + 64 * i, 0, TILE_CPOL);
    t.k[4 * i + 0] = x.x; t.k[4 * i + 1] = x.y; t.k[4 * i + 2] = x.z; t.k[4 * i + 3] = x.w;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int vo = (4 * g + j) * D + n * (D / 16);
    if constexpr (D == 128) {
      const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(rv, vo, 0, TILE_CPOL);
      t.v[2 * j + 0] = x.x; t.v[2 * j + 1] = x.y;
    } else {
      t.v[j] = __builtin_amdgcn_raw_buffer_load_b32(rv, vo, 0, TILE_CPOL);
    }
  }
  if constexpr (WF == TIERKV_WARM_ABSMAX_I8) {
    const uint32_t so = live ? (uint32_t(slot) * uint32_t(p.kv_heads) + uint32_t(kvh)) * 4u : wm.bytes;
    t.mr[0] = __builtin_amdgcn_raw_buffer_load_b32(wm.ks, 0, so, 0);
    t.mr[1] = __builtin_amdgcn_raw_buffer_load_b32(wm.vs, 0, so, 0);
  } else {
    // One load (the slot of a dead step is a clamped list entry, in range,
    // so the load needs no guard).
    // Row a of the (block, head): 16 fp16 values, this lane's tokens 4g .. 4g+3.
    const u32x2 x = *reinterpret_cast<const u32x2*>(wm.row + (tile0 + 4 * g) * 2);
    t.mr[0] = x.x;
    t.mr[1] = x.y;
  }
}

__device__ __forceinline__ float half_of(const uint32_t* pair, int r) {
  const uint32_t w = pair[r >> 1];
  return (r & 1) ? half_hi(w) : half_lo(w);
}

// Per-wave softmax state.  acc holds O^T: acc[s][r] = O[head n][(4g + r) * DS + s]
// scaled by PBOOST and 2^-m_run; l and corr are this lane's partial sums
// over its four tokens (reduced over g at the end).  ocorr is the int8
// codes' offset term summed by the MFMA: 1152 * (the sum of head n's fp16 P
// over all tokens of the tiles), the same in every lane of the head.
template <int D>
struct WaveState {
  f32x4 acc[D / 16];
  float ocorr;
  float m_run;
  float l_part;
  float corr;
};

template <int D>
__device__ __forceinline__ void rescale_state(float m_new, WaveState<D>& ws) {
  const float alpha = (ws.m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(ws.m_run - m_new);
#pragma unroll
  for (int s = 0; s < D / 16; ++s) ws.acc[s] *= alpha;
  ws.ocorr *= alpha;
  ws.l_part *= alpha;
  ws.corr *= alpha;
  ws.m_run = m_new;
}

// Lazy online-softmax update for the four logits x[] of this lane; returns
// p[r] = 2^(x[r] - m_run).  The running maximum is re-based (and the state
// rescaled) only when a logit exceeds it by more than LAZY_T.
//
// With SCORES the block's own statistics are staged per head at stage index
// si (the tile's logical block, or its list position): its maximum
// logit bm and bs = sum_t 2^(x_t - bm), both functions of the block's logits
// alone (a fixed reduction over the 16 tokens), so they do not depend on the
// order in which waves and splits met the blocks.  P is then formed as
// 2^(x - bm) * 2^(bm - m_run).
template <int D, bool SCORES>
__device__ __forceinline__ void softmax_step(const DecodeParams& p, const float* x, float* pr, int lane,
                                             bool head_ok, int b, int qh, int si, float* s_stage,
                                             WaveState<D>& ws) {
  const int g = lane >> 4;
  const float lm = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
  if constexpr (SCORES) {
    float bm = fmaxf(lm, xor16_f(lm));
    bm = fmaxf(bm, xor32_f(bm));
    if (__any(head_ok && bm > ws.m_run + LAZY_T)) {
      rescale_state<D>(fmaxf(ws.m_run, bm), ws);
    }
    const float bmr = (bm == -INFINITY) ? 0.f : bm;
    float e[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) e[r] = __builtin_amdgcn_exp2f(x[r] - bmr);
    const float es = (e[0] + e[1]) + (e[2] + e[3]);
    float bs = es + xor16_f(es);
    bs += xor32_f(bs);
    if (g == 0 && head_ok) {
      if (s_stage) {
        // LDS stage [G][row] of (max, sum) at this tile's stage index (its
        // logical block or its list position); lane n < G is head n.
        const int row = (p.lds_stage == STAGE_LDS_LIST) ? MAX_LIST : p.num_blocks;
        reinterpret_cast<float2*>(s_stage)[(lane & 15) * row + si] = make_float2(bm, bs);
      } else {
        // Workspace stage, read by the finalisation kernel after this launch.
        *reinterpret_cast<float2*>(p.ws_stage + ((int64_t(b) * p.num_heads + qh) * p.num_blocks + si) * 2) =
            make_float2(bm, bs);
      }
    }
    const float f = __builtin_amdgcn_exp2f(bmr - ws.m_run);
#pragma unroll
    for (int r = 0; r < 4; ++r) pr[r] = e[r] * f;
    ws.l_part += es * f;
  } else {
    if (__any(head_ok && lm > ws.m_run + LAZY_T)) {
      float tm = fmaxf(lm, xor16_f(lm));
      tm = fmaxf(tm, xor32_f(tm));
      rescale_state<D>(fmaxf(ws.m_run, tm), ws);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) pr[r] = __builtin_amdgcn_exp2f(x[r] - ws.m_run);
    ws.l_part += (pr[0] + pr[1]) + (pr[2] + pr[3]);
  }
}

__device__ __forceinline__ void mask_tail(float* x, int g, int len) {
  if (len < FBS) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (4 * g + r >= len) x[r] = -INFINITY;
  }
}

template <int D, bool SCORES>
__device__ __forceinline__ void process_hot(const DecodeParams& p, const HotTile<D>& t, int si, int len, int lane,
                                            bool head_ok, int b, int qh, const uint32_t* qv, float* s_stage,
                                            WaveState<D>& ws) {
  constexpr int DS = D / 16;
  constexpr int RW = HotTile<D>::RW;
  // S^T = K Q^T
  f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < DS; ++s)
    sacc = __builtin_amdgcn_mfma_f32_16x16x16f16(as_f16x4(t.k[2 * s], t.k[2 * s + 1]),
                                                 as_f16x4(qv[2 * s], qv[2 * s + 1]), sacc, 0, 0, 0);
  float x[4], pr[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) x[r] = sacc[r] * p.scale_log2;
  mask_tail(x, lane >> 4, len);
  softmax_step<D, SCORES>(p, x, pr, lane, head_ok, b, qh, si, s_stage, ws);
  // O^T += V^T P^T; the A operand of step s is {V[4g + j][n*DS + s]}_j.
  const f16x4 pf = as_f16x4(pack_f16x2(pr[0] * PBOOST, pr[1] * PBOOST), pack_f16x2(pr[2] * PBOOST, pr[3] * PBOOST));
#pragma unroll
  for (int s = 0; s < DS; ++s) {
    const int dw = s >> 1;
    const uint32_t sel = (s & 1) ? 0x07060302u : 0x05040100u;
    const f16x4 av = as_f16x4(perm_b32(t.v[1 * RW + dw], t.v[0 * RW + dw], sel),
                              perm_b32(t.v[3 * RW + dw], t.v[2 * RW + dw], sel));
    ws.acc[s] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, pf, ws.acc[s], 0, 0, 0);
  }
}

template <int D, int WF, bool SCORES>
__device__ __forceinline__ void process_warm(const DecodeParams& p, const WarmTile<D, WF>& t, int si, int len,
                                             int lane, bool head_ok, int b, int qh, const uint32_t* qv, float qsum,
                                             float* s_stage, WaveState<D>& ws) {
  constexpr int DS = D / 16;
  constexpr int RW = WarmTile<D, WF>::RW;
  uint32_t m[WarmTile<D, WF>::NM];
  warm_meta<D, WF>(t, m);
  // S^T = (K + offset) Q^T with the codes as exact fp16 integers.
  f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < DS; ++s) {
    const f16x4 a = (WF == TIERKV_WARM_ABSMAX_I8) ? i8x4_plus1152(t.k[s]) : u8x4_plus1024(t.k[s]);
    sacc = __builtin_amdgcn_mfma_f32_16x16x16f16(a, as_f16x4(qv[2 * s], qv[2 * s + 1]), sacc, 0, 0, 0);
  }
  float x[4], pr[4];
  if constexpr (WF == TIERKV_WARM_ABSMAX_I8) {
    const float c1 = p.scale_log2 * __uint_as_float(m[0]);
    const float c0 = -BIAS_I8 * qsum * c1;
#pragma unroll
    for (int r = 0; r < 4; ++r) x[r] = fmaf(sacc[r], c1, c0);
  } else {
    // s * (S' - (1024 + z) * qsum): the offset is subtracted before the
    // scale, so the cancellation happens between two values of one size.
    const float q1024 = BIAS_U8 * qsum;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      x[r] = (sacc[r] - fmaf(half_of(&m[2], r), qsum, q1024)) * (p.scale_log2 * half_of(&m[0], r));
  }
  mask_tail(x, lane >> 4, len);
  softmax_step<D, SCORES>(p, x, pr, lane, head_ok, b, qh, si, s_stage, ws);

  // O^T += V^T P^T: the A operand of step s holds the four tokens of dim
  // n*DS + s (a byte transpose of the four rows' codes: vt[s]).
  auto transpose_v = [&](uint32_t* vt) {
#pragma unroll
    for (int w4 = 0; w4 < RW; ++w4)
      transpose_bytes4x4(t.v[0 * RW + w4], t.v[1 * RW + w4], t.v[2 * RW + w4], t.v[3 * RW + w4], &vt[4 * w4]);
  };
  uint32_t vt[DS];
  if constexpr (WF == TIERKV_WARM_ABSMAX_I8) {
    const float sv = __uint_as_float(m[1]);
    if (sv <= FOLD_MAX) {
      const float f = PBOOST * sv;
      const f16x4 pf = as_f16x4(pack_f16x2(pr[0] * f, pr[1] * f), pack_f16x2(pr[2] * f, pr[3] * f));
      // The offset 1152 of every code is removed with the same fp16 P values
      // the MFMA multiplies: an A operand of 1152s gives 1152 * sum(P) per
      // head (in every element of its result).
      const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
      ws.ocorr += __builtin_amdgcn_mfma_f32_16x16x16f16(as_f16x4(BIAS_I8_F16X2, BIAS_I8_F16X2), pf, zero4, 0, 0, 0)[0];
#pragma unroll
      for (int s = 0; s < DS; ++s)
        ws.acc[s] = __builtin_amdgcn_mfma_f32_16x16x16f16(
            i8_col_plus1152(t.v[0 * RW + s / 4], t.v[1 * RW + s / 4], t.v[2 * RW + s / 4], t.v[3 * RW + s / 4], s % 4),
            pf, ws.acc[s], 0, 0, 0);
    } else {
      transpose_v(vt);
      // Large V scale: apply it to V (fp16(c * s_v)) so that P stays in range.
      const f16x4 pf = as_f16x4(pack_f16x2(pr[0] * PBOOST, pr[1] * PBOOST), pack_f16x2(pr[2] * PBOOST, pr[3] * PBOOST));
#pragma unroll
      for (int s = 0; s < DS; ++s) {
        const uint32_t w = vt[s];
        const float a0 = float(int8_t(w & 0xffu)) * sv;
        const float a1 = float(int8_t((w >> 8) & 0xffu)) * sv;
        const float a2 = float(int8_t((w >> 16) & 0xffu)) * sv;
        const float a3 = float(int8_t(w >> 24)) * sv;
        ws.acc[s] = __builtin_amdgcn_mfma_f32_16x16x16f16(as_f16x4(pack_f16x2(a0, a1), pack_f16x2(a2, a3)), pf,
                                                          ws.acc[s], 0, 0, 0);
      }
    }
  } else {
    transpose_v(vt);
    // A scale above FOLD_MAX (or a negative or non-finite one) takes the
    // unfolded path: a positive fp16 orders as its bit pattern, and every
    // other pattern compares above FOLD_MAX's.
    const uint32_t smax = max(max(m[4] & 0xffffu, m[4] >> 16), max(m[5] & 0xffffu, m[5] >> 16));
    if (!__any(smax > FOLD_MAX_F16)) {
      // P * PBOOST rounded to fp16, then times the fp16 scale (packed fp16:
      // at most a second rounding of 2^-11 on each P).
      const f16x2 pb01 = as_f16x2(pack_f16x2(pr[0] * PBOOST, pr[1] * PBOOST));
      const f16x2 pb23 = as_f16x2(pack_f16x2(pr[2] * PBOOST, pr[3] * PBOOST));
      const f16x4 pf = as_f16x4(bits_of(pb01 * as_f16x2(m[4])), bits_of(pb23 * as_f16x2(m[5])));
      // The offset (1024 + zero) is removed with the fp16 P values the MFMA
      // multiplies: an A operand whose four k values are this lane's tokens'
      // 1024 + zero (exact fp16 integers) gives sum_t (1024 + zero_t) P_t per
      // head in every element.
      const f16x2 b1024 = {_Float16(BIAS_U8), _Float16(BIAS_U8)};
      const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
      ws.ocorr += __builtin_amdgcn_mfma_f32_16x16x16f16(
          as_f16x4(bits_of(as_f16x2(m[6]) + b1024), bits_of(as_f16x2(m[7]) + b1024)), pf, zero4, 0, 0, 0)[0];
#pragma unroll
      for (int s = 0; s < DS; ++s)
        ws.acc[s] = __builtin_amdgcn_mfma_f32_16x16x16f16(u8x4_plus1024(vt[s]), pf, ws.acc[s], 0, 0, 0);
    } else {
      // (u - zero) * scale per token in fp32, as the reference kernel does.
      float sv[4], zv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sv[r] = half_of(&m[4], r);
        zv[r] = half_of(&m[6], r);
      }
      const f16x4 pf = as_f16x4(pack_f16x2(pr[0] * PBOOST, pr[1] * PBOOST), pack_f16x2(pr[2] * PBOOST, pr[3] * PBOOST));
#pragma unroll
      for (int s = 0; s < DS; ++s) {
        const uint32_t w = vt[s];
        const float a0 = (float(w & 0xffu) - zv[0]) * sv[0];
        const float a1 = (float((w >> 8) & 0xffu) - zv[1]) * sv[1];
        const float a2 = (float((w >> 16) & 0xffu) - zv[2]) * sv[2];
        const float a3 = (float(w >> 24) - zv[3]) * sv[3];
        ws.acc[s] = __builtin_amdgcn_mfma_f32_16x16x16f16(as_f16x4(pack_f16x2(a0, a1), pack_f16x2(a2, a3)), pf,
                                                          ws.acc[s], 0, 0, 0);
      }
    }
  }
}

// Final softmax quantities of one head from the combined base-2 maximum M
// and denominator L of the resident tokens (the accumulator is in PBOOST
// units, L is not).  COLD tokens of the zero-logit mode enter with logit 0
// (tierkv_triton.py:92-102); f rescales the resident accumulator.
template <bool COLD_ZERO>
__device__ __forceinline__ void cold_adjust(float& M, float& L, float& f, float cold_tokens) {
  f = 1.f;
  if (COLD_ZERO && cold_tokens > 0.f) {
    const float M2 = fmaxf(M, 0.f);
    f = (M == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(M - M2);
    L = L * f + cold_tokens * __builtin_amdgcn_exp2f(-M2);
    M = M2;
  }
}

// Combine two (max, sum-relative-to-max) pairs of base-2 softmax statistics.
// Symmetric in its operands bit for bit (max, and one product per operand
// added commutatively), so a butterfly over lanes gives every lane the same
// value and the result depends only on the pairs, not on who combines them.
// Branch-free: selects instead of an early return when both maxima are
// -inf (which leaves the pair as it was), so the butterflies' dependent
// chains carry no branches (the score finalisation: C3 40.56 -> 40.33 us,
// C4 38.46 -> 38.10 us per step).
__device__ __forceinline__ void combine_ms(float& m, float& s, float m2, float s2) {
  const float M = fmaxf(m, m2);
  const float a = (m == -INFINITY) ? 0.f : s * __builtin_amdgcn_exp2f(m - M);
  const float c = (m2 == -INFINITY) ? 0.f : s2 * __builtin_amdgcn_exp2f(m2 - M);
  s = (M == -INFINITY) ? s : a + c;
  m = M;
}

// Value of lane 16 * (lane / 16) + (lane + N) % 16 (DPP row rotate).
template <int N>
__device__ __forceinline__ float row_ror(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + N, 0xf, 0xf, false));
}

// Every lane receives the combination of the wave's 64 (max, sum) pairs, in
// a fixed order: row rotations by 8, 4, 2, 1 (after each, lanes that are
// paired hold bit-identical values because combine_ms is symmetric), then
// the 16- and 32-lane exchanges.
__device__ __forceinline__ void wave_combine_ms(float& m, float& s) {
  combine_ms(m, s, row_ror<8>(m), row_ror<8>(s));
  combine_ms(m, s, row_ror<4>(m), row_ror<4>(s));
  combine_ms(m, s, row_ror<2>(m), row_ror<2>(s));
  combine_ms(m, s, row_ror<1>(m), row_ror<1>(s));
  combine_ms(m, s, xor16_f(m), xor16_f(s));
  combine_ms(m, s, xor32_f(m), xor32_f(s));
}

// One lane's share of a score part (below): its entries j = 0, 1, ...
// (blocks lo + lane + 64 j) in rounds of FOLD_ROUND; a round is reduced by a
// balanced binary tree over its FOLD_ROUND slots and the rounds are combined
// into (m, s) in ascending order.  Slots past the lane's entries, and blocks
// without a tile (max -inf), are the identity (-inf, 0), which combine_ms
// leaves exact, so a round reduced over U < FOLD_ROUND slots (U a power of
// two covering the lane's entries) gives the same bits as the full tree.  The
// tree's levels are independent combines, where a sequential fold would be
// one dependent chain of exponentials per lane.
constexpr int FOLD_ROUND = 16;

template <int U>
__device__ __forceinline__ void fold_round(const float2* e, int live, float& m, float& s) {
  static_assert(U <= FOLD_ROUND && (U & (U - 1)) == 0, "a round is a power of two of at most FOLD_ROUND slots");
  float tm[U], ts[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const bool use = u < live && e[u].x != -INFINITY;
    tm[u] = use ? e[u].x : -INFINITY;
    ts[u] = use ? e[u].y : 0.f;
  }
#pragma unroll
  for (int w2 = 1; w2 < U; w2 *= 2)
#pragma unroll
    for (int u = 0; u < U; u += 2 * w2) combine_ms(tm[u], ts[u], tm[u + w2], ts[u + w2]);
  combine_ms(m, s, tm[0], ts[0]);
}

// Staged statistics of a block that no tile visits: (-inf, -len) for a COLD
// block whose tokens enter the softmax (zero-logit mode), (-inf, 0) for one
// that contributes nothing.
template <bool COLD_ZERO>
__device__ __forceinline__ float2 stage_blank(int st, int len) {
  return make_float2(-INFINITY, (COLD_ZERO && st == COLD) ? -float(len) : 0.f);
}

// Probability sum of a block from its staged (bm, bs) and its head's (M, L)
// (cold_p: the probability of one zero-logit COLD token).
__device__ __forceinline__ float block_score(float2 e, float M, float inv_l, float cold_p) {
  if (e.y < 0.f) return -e.y * cold_p;
  if (e.x != -INFINITY) return e.y * __builtin_amdgcn_exp2f(e.x - M) * inv_l;
  return 0.f;
}

// Score reduction tree of a head's row: `parts` contiguous ranges of
// ceil(nb / parts) blocks, one wave each (lane l folds blocks lo + l,
// lo + l + 64, ... with fold_round, then wave_combine_ms), the parts
// combined in ascending order.  parts = nw / G when the unit's G heads fit
// in its nw waves, else 1; the decode workgroup and the finalisation kernel
// both follow it, so score sums do not depend on the launch's split count.
__host__ __device__ inline int score_parts(int groups, int nw) { return groups <= nw ? nw / groups : 1; }

// The arguments the list build needs first come ahead of the parameter block
// so that they can be preloaded into scalar registers at wave launch.
template <int D, int WF, bool SCORES, bool COLD_ZERO, typename QT, int NW, bool LONG>
__global__ __launch_bounds__(MAX_WAVES * 64) void tiered_decode_kernel(
    const int32_t* __restrict__ a_table, const int32_t* __restrict__ a_states,
    const int32_t* __restrict__ a_lengths, const void* __restrict__ a_q,
    const int32_t* __restrict__ a_seq_nblocks, int32_t a_stride, int32_t a_num_blocks,
    int32_t a_kvh_splits, uint32_t a_split_magic, DecodeParams p) {
  constexpr int DS = D / 16;
  extern __shared__ float s_dyn[];               // [NW][G][D] wave accumulators, then the LDS stage
  __shared__ int4 s_list[MAX_LIST];              // (block, slot, len, state)
  __shared__ int s_wcnt[2][PRE_CHUNKS * MAX_WAVES];   // per (chunk, wave): HOT / WARM counts
  __shared__ int s_wcold[MAX_WAVES];
  __shared__ int s_last;
  __shared__ int s_next[2];                      // next WARM / HOT list position to hand out
  __shared__ int s_prog[MAX_WAVES];              // deterministic launches: tiles taken per wave
  __shared__ float s_m[MAX_WAVES][16];
  __shared__ float s_l[MAX_WAVES][16];
  __shared__ float s_tm[16];                     // score finalisation: per (head, part) max and sum
  __shared__ float s_ts[16];

  const int G = p.groups;
  // kv heads (bits 0-15), splits (bits 16-30) and the XCD placement flag
  // (bit 31, below) share one preloaded argument, so that the split magic
  // (used by the rank) is preloaded too.
  const int a_kv_heads = a_kvh_splits & 0xffff;
  const int splits = int((uint32_t(a_kvh_splits) >> 16) & 0x3fffu);
  const bool det = ((uint32_t(a_kvh_splits) >> 30) & 1u) != 0;
  // Unsplit launches of a batch that is a multiple of the 8 XCDs (bit 31):
  // the hardware deals consecutive workgroups to the XCDs in turn, so
  // workgroup i serves sequence 8 * (s / kv_heads) + i % 8 and kv head
  // s % kv_heads with s = i / 8, and the kv heads of one sequence run on one
  // XCD.  Their per-token scale / zero rows of the reference WARM format
  // share cache lines (four heads' 32-byte rows in a 128-byte line), which
  // that XCD's L2 then fetches once (traffic 1.074x -> 1.002x of ideal at
  // C3), and the sequence's table row is fetched once per XCD.  The flag is
  // decided on the host and the mapping has no branch, so nothing delays
  // the first table loads (a branch here let the compiler place the
  // parameter-block loads and their wait ahead of them: C4 +0.3 us).
  const bool xcd_seq = a_kvh_splits < 0;
  const int u = (int(blockIdx.x) >> (xcd_seq ? 3 : 0)) / splits;   // splits == 1 when xcd_seq
  const int bq = u / a_kv_heads;
  const int b = xcd_seq ? 8 * bq + int(blockIdx.x & 7u) : bq;
  const int kvh = u - bq * a_kv_heads;
  const int split = int(blockIdx.x) % splits;
  const int unit = b * a_kv_heads + kvh;
  const int tid = threadIdx.x;
  constexpr int nthreads = NW * 64;
  constexpr int nw = NW;
  const int lane = tid & 63;
  const int w = tid >> 6;
  // ---- the first table loads leave before anything that needs a kernel
  // argument beyond the preloaded ones (whose wait would hold them back).
  // Long rows: PRE_CHUNKS chunks of nthreads entries; short rows (at most
  // nthreads blocks, which the host guarantees): one entry per thread.  Past
  // the row's end the last entry is re-read and ignored, so the loads need
  // no branch.  The three entries of a block (state, length, slot) are
  // loaded together.
  constexpr int NLD = LONG ? PRE_CHUNKS : 1;
  int st0[NLD], len0[NLD], slot0[NLD];
#pragma unroll
  for (int k = 0; k < NLD; ++k) {
    const int64_t o = int64_t(b) * a_stride + min(k * nthreads + tid, a_num_blocks - 1);
    st0[k] = a_states[o];
    len0[k] = a_lengths[o];
    slot0[k] = a_table[o];
  }
  __builtin_amdgcn_sched_barrier(0);
  // Blocks of this sequence: the per-sequence count is loaded together with
  // the first row chunk and applied afterwards.
  const int nb_ld = a_seq_nblocks ? a_seq_nblocks[b] : a_num_blocks;
  // Per-block score statistics (max, sum) per head (STAGE_* modes above).
  // Nothing the list build does depends on the stage mode, a kernel argument
  // outside the preloaded ones whose load would hold the build up.  A block
  // that no tile will visit gets an entry too (stage_blank), so the staged
  // statistics describe every block below the row's count.  The list build's
  // first pass records the blanks of its entries in blank_bits (8 bits per
  // entry: blank, COLD, length); after the tile loops they go to the LDS
  // block stage, or to the workspace from the split that owns the block
  // (split s: blocks [s * own, (s + 1) * own), so a wave's stores are
  // contiguous).  Later passes (rows beyond PRE_CHUNKS * nthreads blocks;
  // block and workspace stages only) write theirs at once.
  const int own = (a_num_blocks + splits - 1) / splits;
  uint32_t blank_bits = 0;
  auto stage_base = [&]() -> float* {
    return p.ws_stage + (int64_t(b) * p.num_heads + int64_t(kvh) * G) * p.num_blocks * 2;
  };
  auto lds_blank = [&](int idx, int st, int len) {
    float2* const ls = reinterpret_cast<float2*>(s_dyn + NW * G * D);
    for (int h = 0; h < G; ++h) ls[h * p.num_blocks + idx] = stage_blank<COLD_ZERO>(st, len);
  };
  auto store_blank = [&](int idx, int st, int len) {
    float* const gs = stage_base();
    for (int h = 0; h < G; ++h)
      *reinterpret_cast<float2*>(gs + (int64_t(h) * p.num_blocks + idx) * 2) = stage_blank<COLD_ZERO>(st, len);
  };
  auto owned = [&](int idx) { return uint32_t(idx - split * own) < uint32_t(own); };
  // blank: the entry is below the row's count and has no tile.  The pass is
  // uniform; the first pass's bookkeeping is branch-free.
  auto stage_init = [&](bool blank, int idx, int st, int len, int k, bool first_pass) {
    if (first_pass) {
      blank_bits |= blank ? uint32_t(1 | ((st == COLD) ? 2 : 0) | (len << 2)) << (8 * k) : 0u;
    } else if (blank) {
      if (p.lds_stage == STAGE_LDS_BLOCK) lds_blank(idx, st, len);
      else if (owned(idx)) store_blank(idx, st, len);
    }
  };
  // The first pass's blanks: all of them into the LDS block stage, or the
  // owned ones into the workspace stage.
  auto flush_blanks = [&](bool to_lds) {
#pragma unroll
    for (int k = 0; k < NLD; ++k) {
      const uint32_t e = (blank_bits >> (8 * k)) & 0xffu;
      const int idx = k * nthreads + tid;
      if (!(e & 1u)) continue;
      if (to_lds) lds_blank(idx, (e & 2u) ? COLD : HOT, int(e >> 2));
      else if (owned(idx)) store_blank(idx, (e & 2u) ? COLD : HOT, int(e >> 2));
    }
  };
  if (tid == 0) {
    s_next[0] = 0;
    s_next[1] = 0;
    for (int i = 0; i < MAX_WAVES; ++i) s_prog[i] = 0;
  }

  // ---- query: issued right after the first table loads, converted once the
  // list is built.  Its address needs kernel arguments beyond the preloaded
  // ones, so their load overlaps the table loads' round trip.
  const int n = lane & 15;
  const int g = lane >> 4;
  const bool head_ok = n < G;
  const int qh = kvh * G + (head_ok ? n : 0);
  uint4 qraw[D / 32], qraw_h[D / 32];
  auto load_query = [&]() {
    const QT* qrow = reinterpret_cast<const QT*>(a_q) + (int64_t(b) * p.num_heads + qh) * D;
    // WARM K permutation: for load il of a WARM K tile, dims 64il + 16g .. +15.
#pragma unroll
    for (int i = 0; i < D / 32; ++i)
      qraw[i] = *reinterpret_cast<const uint4*>(qrow + 64 * (i >> 1) + 16 * g + 8 * (i & 1));
#pragma unroll
    for (int i = 0; i < D / 32; ++i) qraw_h[i] = *reinterpret_cast<const uint4*>(qrow + 32 * i + 8 * g);
  };

  // ---- this workgroup's share of the resident blocks ------------------------
  // One pass over the table row.  HOT and WARM blocks are ranked separately in
  // logical order; the workgroup keeps rank % splits == split (rows of one
  // pass of the long-row build: a contiguous range of ranks), HOT entries at
  // list positions [0, nhot) from the front, WARM entries from the back
  // (position MAX_LIST - 1 - k for the k-th).  The first pass ranks the
  // entries loaded at the kernel's start.  COLD tokens (zero-logit mode) are
  // counted per thread and reduced per wave.
  int nb = a_num_blocks;
  int seen_hot = 0, seen_warm = 0;
  int cold_part = 0;
  int bad = 0;   // error bits of this lane's entries (kept in a vector register)
  const uint32_t hot_cap = uint32_t(min(p.hot_slots, int64_t(0x7fffffff)));
  const uint32_t warm_cap = uint32_t(min(p.warm_slots, int64_t(0x7fffffff)));
  // Whether rank r belongs to this split (r % splits == split), and its list
  // position q = r / splits: one multiply-high by ceil(2^32 / splits) and a
  // correction (exact while r * splits < 2^32, which the host checks).
  // x / splits for 0 <= x <= num_blocks * splits (the same multiply-high).
  auto div_splits = [&](int x) -> int {
    if (splits == 1) return x;
    if (a_split_magic != 0) {
      uint32_t qq = __umulhi(uint32_t(x), a_split_magic);
      if (qq * uint32_t(splits) > uint32_t(x)) qq -= 1u;
      return int(qq);
    }
    return int(uint32_t(x) / uint32_t(splits));
  };
  // This workgroup's HOT / WARM entry counts when it owns contiguous rank
  // ranges (rows of one pass of the long-row build), else -1.
  int own_h = -1, own_w = -1;
  auto mine = [&](int r, int& q) -> bool {
    if (splits == 1) {
      q = r;
      return true;
    }
    if (a_split_magic != 0) {
      uint32_t qq = __umulhi(uint32_t(r), a_split_magic);
      if (qq * uint32_t(splits) > uint32_t(r)) qq -= 1u;
      q = int(qq);
    } else {
      q = r / splits;
    }
    return r - q * splits == split;
  };
  if constexpr (LONG) {
    // Long rows: PRE_CHUNKS chunks of nthreads entries are loaded before any
    // is ranked, so a row of up to PRE_CHUNKS * nthreads blocks costs one
    // memory round trip and one barrier (the long-context rows of 2048
    // blocks included); the (chunk, wave) counts are scanned across lanes.
    // The first pass is written out before the loop over further passes, so
    // that no wait at the loop's head holds its loads behind the query's.
    using Chunks = int[PRE_CHUNKS];
    const bool one_pass = a_num_blocks <= PRE_CHUNKS * nthreads;
    auto load_chunks = [&](int c0, Chunks& st, Chunks& len, Chunks& slot) {
      // Past the row's end the last entry is re-read and ignored: the loads
      // need no per-lane branch.
  #pragma unroll
      for (int k = 0; k < PRE_CHUNKS; ++k) {
        const int idx = min(c0 + k * nthreads + tid, a_num_blocks - 1);
        const int64_t o = int64_t(b) * a_stride + idx;
        st[k] = a_states[o];
        len[k] = a_lengths[o];
        slot[k] = a_table[o];
      }
    };
    auto rank_chunks = [&](int c0, Chunks& st, Chunks& len, Chunks& slot) {
      // Class of each entry: 1 HOT, 2 WARM, 0 neither.  It is kept per lane
      // and the ballots are taken again after the barrier, so no lane masks
      // stay live across it.
      int cls[PRE_CHUNKS];
  #pragma unroll
      for (int k = 0; k < PRE_CHUNKS; ++k) {
        const bool in_row = c0 + k * nthreads + tid < nb;
        len[k] = min(max(len[k], 0), FBS);
        const bool tiered = st[k] == HOT || st[k] == WARM;
        const bool slot_ok = uint32_t(slot[k]) < ((st[k] == HOT) ? hot_cap : warm_cap);
        const bool use = in_row && tiered && slot_ok && len[k] > 0;
        cls[k] = use ? ((st[k] == HOT) ? 1 : 2) : 0;
        bad |= (in_row && tiered && !slot_ok && len[k] > 0) ? 1 : 0;
        bad |= (in_row && !tiered && st[k] != COLD) ? 2 : 0;
        if (COLD_ZERO) cold_part += (in_row && st[k] == COLD) ? len[k] : 0;
        if (SCORES) stage_init(in_row && cls[k] == 0, c0 + k * nthreads + tid, st[k], len[k], k, c0 == 0);
        const int nh = __popcll(__ballot(cls[k] == 1));
        const int nwm = __popcll(__ballot(cls[k] == 2));
        if (lane == 0) {
          s_wcnt[0][k * nw + w] = nh;
          s_wcnt[1][k * nw + w] = nwm;
        }
      }
      __syncthreads();
      // Exclusive prefix of the (chunk, wave) counts in logical order: lane j
      // holds count j, a wave-wide scan gives every wave every base.
      constexpr int nj = PRE_CHUNKS * nw;
      const int ch = (lane < nj) ? s_wcnt[0][lane] : 0;
      const int cw = (lane < nj) ? s_wcnt[1][lane] : 0;
      const int ih = wave_inclusive_scan(ch);
      const int iw = wave_inclusive_scan(cw);
      if (one_pass) {
        // Rows of one pass: split s owns the contiguous ranks
        // [tot * s / splits, tot * (s + 1) / splits) of each tier.  Lane j
        // holds chunk j's bases relative to this workgroup's ranges; the
        // chunks are ranked without branches, so their scalar reads overlap.
        const int tot_h = __builtin_amdgcn_readlane(ih, nj - 1);
        const int tot_w = __builtin_amdgcn_readlane(iw, nj - 1);
        // x / splits without branches: a row of one pass has num_blocks *
        // splits < 2^32, so the multiply-high is exact whenever splits > 1.
        auto div_one = [&](int x) -> int {
          uint32_t qq = __umulhi(uint32_t(x), a_split_magic);
          qq -= (qq * uint32_t(splits) > uint32_t(x)) ? 1u : 0u;
          return splits == 1 ? x : int(qq);
        };
        const int lo_h = div_one(tot_h * split), lo_w = div_one(tot_w * split);
        own_h = div_one(tot_h * (split + 1)) - lo_h;
        own_w = div_one(tot_w * (split + 1)) - lo_w;
        const int rh = ih - ch - lo_h;
        const int rw = iw - cw - lo_w;
        const int wu = uniform(w);
  #pragma unroll
        for (int k = 0; k < PRE_CHUNKS; ++k) {
          const int hb = __builtin_amdgcn_readlane(rh, k * nw + wu);
          const int wb = __builtin_amdgcn_readlane(rw, k * nw + wu);
          const uint64_t mh = __ballot(cls[k] == 1);
          const uint64_t mw = __ballot(cls[k] == 2);
          const bool is_hot = cls[k] == 1;
          const uint64_t m = is_hot ? mh : mw;
          const int q = int(__builtin_amdgcn_mbcnt_hi(uint32_t(m >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(m), 0u))) +
                        (is_hot ? hb : wb);
          if (cls[k] != 0 && uint32_t(q) < uint32_t(is_hot ? own_h : own_w)) {
            const int idx = k * nthreads + tid;
            const int pos = is_hot ? q : MAX_LIST - 1 - q;
            s_list[pos] = make_int4(idx, slot[k], len[k], pos);
          }
        }
        return;
      }
      const uint64_t below = (1ull << lane) - 1ull;
  #pragma unroll
      for (int k = 0; k < PRE_CHUNKS; ++k) {
        const int j = uniform(k * nw + w);
        const int hb = seen_hot + __builtin_amdgcn_readlane(ih - ch, j);
        const int wb = seen_warm + __builtin_amdgcn_readlane(iw - cw, j);
        const int idx = c0 + k * nthreads + tid;
        const uint64_t mh = __ballot(cls[k] == 1);
        const uint64_t mw = __ballot(cls[k] == 2);
        // One rank and one list write per entry, whichever its tier (the
        // wave runs both tiers' lanes at once).
        const bool is_hot = cls[k] == 1;
        const int r = is_hot ? hb + __popcll(mh & below) : wb + __popcll(mw & below);
        int q;
        if (cls[k] != 0 && mine(r, q)) {
          const int pos = is_hot ? q : MAX_LIST - 1 - q;
          s_list[pos] = make_int4(idx, slot[k], len[k], pos);
        }
      }
      seen_hot += __builtin_amdgcn_readlane(ih, 63);
      seen_warm += __builtin_amdgcn_readlane(iw, 63);
    };
    load_query();
    __builtin_amdgcn_sched_barrier(0);   // every load in flight before any use
    nb = uniform(min(max(nb_ld, 0), a_num_blocks));
    rank_chunks(0, st0, len0, slot0);
    for (int c0 = PRE_CHUNKS * nthreads; c0 < a_num_blocks; c0 += PRE_CHUNKS * nthreads) {
      __syncthreads();   // s_wcnt is reused
      int st[PRE_CHUNKS], len[PRE_CHUNKS], slot[PRE_CHUNKS];
      load_chunks(c0, st, len, slot);
      __builtin_amdgcn_sched_barrier(0);
      rank_chunks(c0, st, len, slot);
    }
  } else {
    // Short rows: one entry per thread, classified without branches (a
    // branch would let the compiler sink a table load into it, after the
    // query loads); the per-wave counts are summed from LDS.
    const int idx = tid;
    load_query();
    __builtin_amdgcn_sched_barrier(0);   // every load in flight before any use
    nb = uniform(min(max(nb_ld, 0), a_num_blocks));
    const int st = st0[0];
    const int len = min(max(len0[0], 0), FBS);
    const int slot = slot0[0];
    const bool in_row = idx < nb;
    const bool tiered = st == HOT || st == WARM;
    const bool slot_ok = uint32_t(slot) < ((st == HOT) ? hot_cap : warm_cap);
    const bool use = in_row && tiered && slot_ok && len > 0;
    const bool hot = use && st == HOT;
    const bool warm = use && st == WARM;
    bad |= (in_row && tiered && !slot_ok && len > 0) ? 1 : 0;
    bad |= (in_row && !tiered && st != COLD) ? 2 : 0;
    if (COLD_ZERO) cold_part += (in_row && st == COLD) ? len : 0;
    if (SCORES) stage_init(in_row && !use, idx, st, len, 0, true);
    const uint64_t mh = __ballot(hot);
    const uint64_t mw = __ballot(warm);
    if (lane == 0) {
      s_wcnt[0][w] = __popcll(mh);
      s_wcnt[1][w] = __popcll(mw);
    }
    __syncthreads();
    int hb = 0, wb = 0;
#pragma unroll
    for (int i = 0; i < nw; ++i) {
      const int ch = s_wcnt[0][i], cw = s_wcnt[1][i];
      hb += (i < w) ? ch : 0;
      wb += (i < w) ? cw : 0;
      seen_hot += ch;
      seen_warm += cw;
    }
    const uint64_t below = (1ull << lane) - 1ull;
    const int r = hot ? hb + __popcll(mh & below) : wb + __popcll(mw & below);
    int q;
    if ((hot || warm) && mine(r, q)) {
      const int pos = hot ? q : MAX_LIST - 1 - q;
      s_list[pos] = make_int4(idx, slot, len, pos);
    }
  }
  if (COLD_ZERO) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) cold_part += __shfl_xor(cold_part, m, 64);
    if (lane == 0) s_wcold[w] = cold_part;
  }
  __syncthreads();
  const int nhot = uniform(own_h >= 0 ? own_h : (seen_hot > split) ? (seen_hot - split + splits - 1) / splits : 0);
  const int nwarm = uniform(own_w >= 0 ? own_w : (seen_warm > split) ? (seen_warm - split + splits - 1) / splits : 0);

  // ---- query (fp16) and its per-head sum ------------------------------------
  // qv: dims 64(i/2) + 16g + 8(i%2) .. +7 in word group i (the WARM K
  // permutation), qvh: dims 32i + 8g .. +7
  // (the HOT K permutation); the same fp16 values in two orders.
  uint32_t qv[D / 8], qvh[D / 8];
  float qsum = 0.f;
  {
    auto to_f16x2 = [&](uint32_t wd) -> uint32_t {
      uint32_t h2;
      if constexpr (std::is_same<QT, __half>::value) {
        h2 = wd;
      } else {
        h2 = pack_f16x2(__uint_as_float(wd << 16), __uint_as_float(wd & 0xffff0000u));
      }
      return head_ok ? h2 : 0u;
    };
#pragma unroll
    for (int i = 0; i < D / 32; ++i) {
      const uint32_t wd[4] = {qraw[i].x, qraw[i].y, qraw[i].z, qraw[i].w};
      const uint32_t wh[4] = {qraw_h[i].x, qraw_h[i].y, qraw_h[i].z, qraw_h[i].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t h2 = to_f16x2(wd[k]);
        qv[4 * i + k] = h2;
        qvh[4 * i + k] = to_f16x2(wh[k]);
        qsum += half_lo(h2) + half_hi(h2);
      }
    }
    qsum += shfl_xor_f(qsum, 16);
    qsum += shfl_xor_f(qsum, 32);
  }

  // ---- per-wave tile loops -------------------------------------------------
  // The list holds this workgroup's HOT entries at positions [0, nhot) and its
  // WARM entries at MAX_LIST - 1 - [0, nwarm).  Waves take positions from two LDS counters
  // (WARM first, then HOT), one tile at a time: the SIMD arbiter favours the
  // older of the two waves it hosts, so a static split would leave the younger
  // waves finishing several tiles late.  Each wave keeps NBW (NBH) tiles of a
  // register pipeline in flight.  Every step issues its load unconditionally
  // (a position past the end reads one cache line for the whole wave and is
  // never processed) and the loops leave only through their latch, so the
  // compiler's wait counts stay exact across iterations.
  // Score statistics: staged by list position (.w) with the list stage, else
  // by logical block (.x).
  const int stage_mode = SCORES ? p.lds_stage : STAGE_GLOBAL;
  const bool list_stage = SCORES && stage_mode == STAGE_LDS_LIST;
  float* const s_stage = (SCORES && stage_mode != STAGE_GLOBAL) ? s_dyn + NW * G * D : nullptr;
  auto stage_index = [&](const int4& e) { return uniform(list_stage ? e.w : e.x); };
  WaveState<D> st;
#pragma unroll
  for (int s = 0; s < DS; ++s) st.acc[s] = f32x4{0.f, 0.f, 0.f, 0.f};
  st.m_run = -INFINITY;
  st.l_part = 0.f;
  st.corr = 0.f;
  st.ocorr = 0.f;

  // Tile hand-out.  By default a wave takes the next list position of the
  // tier from an LDS counter when it frees up.  Deterministic launches give
  // wave w the positions w, w + nw, ... of the WARM list and nw - 1 - w,
  // 2 nw - 1 - w, ... of the HOT list (so that the waves left with one more
  // WARM tile do not also get one more HOT tile): the order of every wave's
  // accumulation is then fixed.  The two waves of a SIMD (w and w ^ 4) would
  // otherwise progress unevenly -- the SIMD's arbiter favours the older one
  // -- so the one behind raises its issue priority after every hand-out.
  // The tile loops are instantiated once per hand-out (one uniform branch
  // here): a check of the mode inside the loops cost the default hand-out
  // 0.7 us at C3.
  auto tile_loops = [&](auto DET) {
    int kc0 = 0, kc1 = 0;
    auto grab = [&](int c) -> int {
      if constexpr (decltype(DET)::value) {
        const int k = c ? kc1++ : kc0++;
        if constexpr (NW == 8) {
          if (lane == 0) s_prog[w] = kc0 + kc1;
          if (uniform(s_prog[w ^ 4]) > kc0 + kc1) __builtin_amdgcn_s_setprio(1);
          else __builtin_amdgcn_s_setprio(0);
        }
        return (c ? nw - 1 - w : w) + nw * k;
      } else {
        int v = 0;
        if (lane == 0) v = atomicAdd(&s_next[c], 1);
        return uniform(v);
      }
    };
    constexpr int NBH = TIERKV_NBH;
    constexpr int NBW = TIERKV_NBW;
    HotTile<D> th[NBH];
    int4 eh[NBH];
    bool lh[NBH];
    int4 hne = make_int4(0, 0, 0, 0);   // next HOT entry to load and whether it is live
    bool hnl = false;
    if (nhot > 0) {
      int gi = grab(1);
      hne = s_list[min(gi, nhot - 1)];
      hnl = gi < nhot;
#pragma unroll
      for (int k = 0; k < NBH - 1; ++k) {
        eh[k] = hne;
        lh[k] = hnl;
        load_hot<D>(p, kvh, uniform(hne.y), lane, th[k], hnl);
        __builtin_amdgcn_sched_barrier(0);
        gi = grab(1);
        hne = s_list[min(gi, nhot - 1)];
        hnl = gi < nhot;
      }
    }
    if (nwarm > 0) {
      const WarmMeta<WF> wm = warm_meta_setup<WF>(p, lane);
      WarmTile<D, WF> tw[NBW];
      int4 ew[NBW];
      bool lw[NBW];
      int gi = grab(0);
      int4 ne = s_list[MAX_LIST - 1 - min(gi, nwarm - 1)];
      bool nl = gi < nwarm;
#pragma unroll
      for (int k = 0; k < NBW - 1; ++k) {
        ew[k] = ne;
        lw[k] = nl;
        load_warm<D, WF>(p, kvh, uniform(ne.y), lane, wm, tw[k], nl);
        __builtin_amdgcn_sched_barrier(0);
        gi = grab(0);
        ne = s_list[MAX_LIST - 1 - min(gi, nwarm - 1)];
        nl = gi < nwarm;
      }
      do {
#pragma unroll
        for (int k = 0; k < NBW; ++k) {
          const int kn = (k + NBW - 1) % NBW;
          ew[kn] = ne;
          lw[kn] = nl;
          load_warm<D, WF>(p, kvh, uniform(ne.y), lane, wm, tw[kn], nl);
          __builtin_amdgcn_sched_barrier(0);
          gi = grab(0);
          ne = s_list[MAX_LIST - 1 - min(gi, nwarm - 1)];
          nl = gi < nwarm;
          if (lw[k])
            process_warm<D, WF, SCORES>(p, tw[k], stage_index(ew[k]), uniform(ew[k].z), lane, head_ok, b, qh, qv,
                                        qsum, s_stage, st);
        }
      } while (lw[0]);   // buffer 0 holds the next tile; positions are handed out in order
    }
    if (nhot > 0) {
      do {
#pragma unroll
        for (int k = 0; k < NBH; ++k) {
          const int kn = (k + NBH - 1) % NBH;
          eh[kn] = hne;
          lh[kn] = hnl;
          load_hot<D>(p, kvh, uniform(hne.y), lane, th[kn], hnl);
          __builtin_amdgcn_sched_barrier(0);
          const int gi = grab(1);
          hne = s_list[min(gi, nhot - 1)];
          hnl = gi < nhot;
          if (lh[k])
            process_hot<D, SCORES>(p, th[k], stage_index(eh[k]), uniform(eh[k].z), lane, head_ok, b, qh, qvh,
                                   s_stage, st);
        }
      } while (lh[0]);
    }
  };
  if (det) tile_loops(std::true_type{});
  else tile_loops(std::false_type{});

  // Error word: bit 1, a resident block with an out-of-range slot (skipped);
  // bit 2, a state that is none of HOT, WARM, COLD.  Reported after the tile
  // loops so that its pointer's kernel-argument load stays off the list
  // build's path.
  if (bad) atomicOr(p.ws_err, bad);

  // ---- merge the waves in LDS (one barrier) ----------------------------------
  float l = st.l_part + shfl_xor_f(st.l_part, 16);
  l += shfl_xor_f(l, 32);
  float corr = st.corr + shfl_xor_f(st.corr, 16);
  corr += shfl_xor_f(corr, 32) + st.ocorr;
  float* s_acc = s_dyn;   // [nw][G][D]
  if (head_ok) {
    if (g == 0) {
      s_m[w][n] = st.m_run;
      s_l[w][n] = l;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int s = 0; s < DS; ++s) s_acc[(w * G + n) * D + (4 * g + r) * DS + s] = st.acc[s][r] - corr;
  }
  if constexpr (SCORES) {
    // The first pass's blanks into the LDS block stage.
    if (stage_mode == STAGE_LDS_BLOCK) flush_blanks(true);
    __builtin_amdgcn_s_waitcnt(0);   // this wave's per-block statistics are stored
  }
  __syncthreads();
  float cold_tokens = 0.f;
  if (COLD_ZERO) {
#pragma unroll
    for (int i = 0; i < nw; ++i) cold_tokens += float(s_wcold[i]);
  }
  // (M, L) of head h over this workgroup's waves and each wave's weight
  // 2^(m_w - M) (0 for a wave that saw no token).  The loops are unrolled so
  // that all LDS reads are in flight together.
  auto wave_ml = [&](int h, float& M, float& L, float* fw) {
    float mw[NW];
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) mw[ww] = s_m[ww][h];
    M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, mw[ww]);
    L = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      fw[ww] = (mw[ww] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(mw[ww] - M);
      L += s_l[ww][h] * fw[ww];
    }
  };
  auto wave_acc = [&](int i, const float* fw) {
    float A = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) A += s_acc[ww * G * D + i] * fw[ww];
    return A;
  };
  QT* out = reinterpret_cast<QT*>(p.out) + (int64_t(b) * p.num_heads + kvh * G) * D;

  // Per-block probability sums of this unit's heads (tierkv_triton.py:121-145)
  // from the staged per-block (bm, bs) pairs.  Each head's maximum M and
  // denominator L over its blocks are reduced in a fixed order: the head's
  // row is cut into `parts` contiguous ranges (one wave each), every lane
  // folds its blocks in ascending order, the wave combines its lanes in a
  // fixed order (wave_combine_ms), and the parts are combined in ascending
  // order.  So score_sums
  // are the same bits on every launch over the same inputs, whatever order
  // the tiles were processed in (the labels ranked from them are
  // reproducible); the attention output keeps its own (M, L).
  // score = bs * 2^(bm - M) / L, or len * 2^-M / L for a COLD block of the
  // zero-logit mode.  A lane's entries of a part (up to 16) are loaded
  // together and, when the wave's only part fits in one such round, kept in
  // registers for the second pass.  The barrier between the passes orders
  // LDS only, so that no wave waits there for its output stores.
  auto finalize_scores = [&]() {
    const int stride = int(p.table_stride);
    const int parts = score_parts(G, nw);
    const int ntask = G * parts;
    const int chunk = (nb + parts - 1) / parts;
    auto entry = [&](int h, int blk) -> float2 {
      return reinterpret_cast<const float2*>(s_stage)[h * p.num_blocks + blk];
    };
    // U entries per lane per round; the caller picks the smallest U that
    // covers a part in one round (rows up to 64 * U blocks per part), else
    // U = FOLD_ROUND.
    auto run = [&](auto u_const) {
      constexpr int U = decltype(u_const)::value;
      const bool reuse = ntask <= nw && chunk <= 64 * U;
      float2 kept[U];
      for (int t = w; t < ntask; t += nw) {
        const int h = t / parts;
        const int lo = (t - h * parts) * chunk;
        const int hi = min(nb, lo + chunk);
        float m = -INFINITY, sum = 0.f;
        for (int c0 = lo; c0 < hi; c0 += U * 64) {
#pragma unroll
          for (int u = 0; u < U; ++u) kept[u] = entry(h, min(c0 + u * 64 + lane, hi - 1));
          fold_round<U>(kept, (hi - c0 - lane + 63) / 64, m, sum);
        }
        wave_combine_ms(m, sum);
        if (lane == 0) {
          s_tm[t] = m;
          s_ts[t] = sum;
        }
      }
      lds_barrier();
      for (int t = w; t < ntask; t += nw) {
        const int h = t / parts;
        const int k0 = t - h * parts;
        float M = -INFINITY, L = 0.f;
        for (int k = 0; k < parts; ++k) combine_ms(M, L, s_tm[h * parts + k], s_ts[h * parts + k]);
        float f;
        cold_adjust<COLD_ZERO>(M, L, f, cold_tokens);
        const float inv_l = (L > 0.f) ? 1.f / L : 0.f;
        const float cold_p = COLD_ZERO ? __builtin_amdgcn_exp2f(-M) * inv_l : 0.f;
        float* dst = p.score_sums + (int64_t(b) * p.num_heads + kvh * G + h) * p.table_stride;
        // Part k writes blocks [min(k * chunk, nb), min((k + 1) * chunk, nb));
        // the last part also writes the zeros of [nb, stride).
        const int lo = min(k0 * chunk, nb);
        const int hi_nb = min(nb, (k0 + 1) * chunk);
        const int hi = (k0 == parts - 1) ? stride : hi_nb;
        for (int c0 = lo; c0 < hi; c0 += U * 64) {
          if (!reuse) {
#pragma unroll
            for (int u = 0; u < U; ++u) kept[u] = entry(h, min(c0 + u * 64 + lane, max(hi_nb - 1, 0)));
          }
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int blk = c0 + u * 64 + lane;
            if (blk >= hi) continue;
            dst[blk] = (blk < hi_nb) ? block_score(kept[u], M, inv_l, cold_p) : 0.f;
          }
        }
      }
    };
    if (chunk <= 128) run(std::integral_constant<int, 2>{});
    else if (chunk <= 256) run(std::integral_constant<int, 4>{});
    else if (chunk <= 512) run(std::integral_constant<int, 8>{});
    else run(std::integral_constant<int, FOLD_ROUND>{});
  };

  if (splits == 1) {
    for (int i = tid; i < G * D; i += nthreads) {
      const int h = i / D;
      float M, L, f, fw[NW];
      wave_ml(h, M, L, fw);
      const float A = wave_acc(i, fw);
      cold_adjust<COLD_ZERO>(M, L, f, cold_tokens);
      out[i] = from_f32<QT>((L > 0.f) ? A * f / (L * PBOOST) : 0.f);
    }
    if (SCORES && stage_mode == STAGE_LDS_BLOCK) finalize_scores();
    if (SCORES && stage_mode == STAGE_GLOBAL) flush_blanks(false);
    return;
  }

  // ---- splits: publish the partial, the last workgroup merges -----------------
  for (int i = tid; i < G * D; i += nthreads) {
    const int h = i / D;
    float M, L, fw[NW];
    wave_ml(h, M, L, fw);
    const int64_t pi = (int64_t(unit) * splits + split) * G + h;
    store_dev(p.ws_acc + pi * D + (i - h * D), wave_acc(i, fw));
    if (i - h * D == 0) {
      store_dev(p.ws_ml + pi * 2 + 0, M);
      store_dev(p.ws_ml + pi * 2 + 1, L);
    }
  }
  // Every wave's device-coherent stores complete before the arrival is counted.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    uint32_t* cnt = p.ws_cnt + unit;
    const bool last = arrive(cnt) == uint32_t(splits - 1);
    if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last ? 1 : 0;
  }
  // Score launches: the statistics this workgroup staged in LDS (by list
  // position) go to the workspace by logical block, and the blanks of the
  // blocks it owns with them, for the finalisation kernel that runs after
  // this launch (no wait covers these stores; the last workgroup issues them
  // after its merge, whose loads would otherwise wait behind them).
  auto flush_stage = [&]() {
    if (list_stage) {
      float* const gs = stage_base();
      const int nlist = nhot + nwarm;
      for (int i = tid; i < G * nlist; i += nthreads) {
        const int h = i / nlist;
        const int j = i - h * nlist;
        const int4 e = (j < nhot) ? s_list[j] : s_list[MAX_LIST - 1 - (j - nhot)];
        *reinterpret_cast<float2*>(gs + (int64_t(h) * p.num_blocks + e.x) * 2) =
            reinterpret_cast<const float2*>(s_stage)[h * MAX_LIST + e.w];
      }
    }
    if (SCORES) flush_blanks(false);
  };
  __syncthreads();
  if (!s_last) {
    flush_stage();
    return;
  }
  // Log-sum-exp merge of the splits' partials (tierkv_triton.py:231-264).
  // Each output element loads every split's (m, l, acc) at once (MERGE_UNROLL
  // splits per round trip) and merges them in registers.
  for (int i = tid; i < G * D; i += nthreads) {
    const int h = i / D;
    const int d = i - h * D;
    float M = -INFINITY, L = 0.f, A = 0.f;
    for (int sp0 = 0; sp0 < splits; sp0 += MERGE_UNROLL) {
      float av[MERGE_UNROLL], mv[MERGE_UNROLL], lv[MERGE_UNROLL];
#pragma unroll
      for (int k = 0; k < MERGE_UNROLL; ++k) {
        const int64_t pi = (int64_t(unit) * splits + min(sp0 + k, splits - 1)) * G + h;
        av[k] = load_dev(p.ws_acc + pi * D + d);
        mv[k] = load_dev(p.ws_ml + pi * 2);
        lv[k] = load_dev(p.ws_ml + pi * 2 + 1);
      }
      float Mn = M;
#pragma unroll
      for (int k = 0; k < MERGE_UNROLL; ++k)
        if (sp0 + k < splits) Mn = fmaxf(Mn, mv[k]);
      if (Mn != -INFINITY) {
        const float rescale = (M == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(M - Mn);
        A *= rescale;
        L *= rescale;
#pragma unroll
        for (int k = 0; k < MERGE_UNROLL; ++k) {
          if (sp0 + k < splits && mv[k] != -INFINITY) {
            const float wgt = __builtin_amdgcn_exp2f(mv[k] - Mn);
            A += av[k] * wgt;
            L += lv[k] * wgt;
          }
        }
        M = Mn;
      }
    }
    float f;
    cold_adjust<COLD_ZERO>(M, L, f, cold_tokens);
    out[i] = from_f32<QT>((L > 0.f) ? A * f / (L * PBOOST) : 0.f);
  }
  flush_stage();
}

// --------------------------------------------------------------------------
// Per-block probability sums of launches whose statistics are staged in the
// workspace (split launches, rows too long for the LDS stage):
// tierkv_triton.py:121-145 from the staged (bm, bs) pairs, which the decode
// launch wrote for every block below each row's count (resident blocks by
// the split that visited them, the others as stage_blank).  One workgroup of
// eight waves per (sequence, q head) row: the row's pairs are loaded into
// LDS by all waves (rows up to FIN_LDS_BLOCKS; longer ones are folded from
// the workspace), the head's (M, L) is reduced along the score tree
// (score_parts: one wave per part, as in the decode workgroup's own
// finalisation, so the sums do not depend on the split count), and every
// thread writes scores.  COLD tokens (zero-logit mode) are read back from
// the blanks and added in integers.  The row is written up to the table
// stride (zeros past the sequence's block count).
// --------------------------------------------------------------------------
// 1024 threads per row: the row's loads and writes spread over sixteen waves
// (C4 with scores: 38.8 -> 38.4 us per step against 512 threads).
constexpr int FIN_THREADS = 1024;
constexpr int FIN_LDS_BLOCKS = 4096;

// All arguments fit the preloaded kernel-argument registers, so the row's
// loads need no kernel-argument fetch; they do not wait for the sequence's
// block count either (the row is read up to num_blocks).
template <bool COLD_ZERO>
__global__ __launch_bounds__(FIN_THREADS) void finalize_scores_kernel(const float* __restrict__ ws_stage,
                                                                      float* __restrict__ score_sums,
                                                                      const int32_t* __restrict__ seq_nblocks,
                                                                      int32_t num_heads, int32_t num_blocks,
                                                                      int32_t stride, int32_t parts) {
  extern __shared__ float2 s_row[];   // [num_blocks] when num_blocks <= FIN_LDS_BLOCKS
  __shared__ float s_pm[MAX_WAVES], s_ps[MAX_WAVES];
  __shared__ int s_pc[MAX_WAVES];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int b = int(blockIdx.x) / num_heads;
  const int h = int(blockIdx.x) - b * num_heads;
  const float2* stage = reinterpret_cast<const float2*>(ws_stage + (int64_t(b) * num_heads + h) * num_blocks * 2);
  const int nb_ld = seq_nblocks ? seq_nblocks[b] : num_blocks;   // used after the row's loads
  const bool in_lds = num_blocks <= FIN_LDS_BLOCKS;
  if (in_lds) {
    constexpr int K = FIN_LDS_BLOCKS / FIN_THREADS;
    float2 v[K];
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (k * FIN_THREADS < num_blocks) v[k] = stage[min(k * FIN_THREADS + tid, num_blocks - 1)];
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (k * FIN_THREADS + tid < num_blocks) s_row[k * FIN_THREADS + tid] = v[k];
  }
  const int nb = min(max(nb_ld, 0), num_blocks);
  if (in_lds) __syncthreads();
  auto entry = [&](int blk) -> float2 { return in_lds ? s_row[blk] : stage[blk]; };

  // This wave's part of the tree (waves w >= parts have none).
  const int chunk = (nb + parts - 1) / parts;
  const int lo = (w < parts) ? min(w * chunk, nb) : nb;
  const int hi = min(nb, lo + chunk);
  float m = -INFINITY, sum = 0.f;
  int cold = 0;
  constexpr int U = FOLD_ROUND;
  for (int c0 = lo; c0 < hi; c0 += U * 64) {
    float2 e[U];
#pragma unroll
    for (int u = 0; u < U; ++u) e[u] = entry(min(c0 + u * 64 + lane, hi - 1));
    fold_round<U>(e, (hi - c0 - lane + 63) / 64, m, sum);
#pragma unroll
    for (int u = 0; u < U; ++u)
      cold += (COLD_ZERO && c0 + u * 64 + lane < hi && e[u].y < 0.f) ? int(-e[u].y) : 0;
  }
  wave_combine_ms(m, sum);
  if (COLD_ZERO) {
#pragma unroll
    for (int k = 32; k >= 1; k >>= 1) cold += __shfl_xor(cold, k, 64);
  }
  if (lane == 0 && w < parts) {
    s_pm[w] = m;
    s_ps[w] = sum;
    s_pc[w] = cold;
  }
  __syncthreads();
  float M = -INFINITY, L = 0.f;
  int cold_total = 0;
  for (int k = 0; k < parts; ++k) {
    combine_ms(M, L, s_pm[k], s_ps[k]);
    cold_total += s_pc[k];
  }
  float f;
  cold_adjust<COLD_ZERO>(M, L, f, float(cold_total));
  const float inv_l = (L > 0.f) ? 1.f / L : 0.f;
  const float cold_p = COLD_ZERO ? __builtin_amdgcn_exp2f(-M) * inv_l : 0.f;

  float* dst = score_sums + (int64_t(b) * num_heads + h) * stride;
  for (int blk = tid; blk < stride; blk += FIN_THREADS)
    dst[blk] = (blk < nb) ? block_score(entry(blk), M, inv_l, cold_p) : 0.f;
}

// --------------------------------------------------------------------------
// Generic path: one wave per (sequence, q head); the reference kernel's
// structure (per-block loop, online softmax, optional second score pass).
// --------------------------------------------------------------------------

template <typename QT, int WF>
__device__ __forceinline__ void generic_kv(const DecodeParams& p, int state, int64_t slot, int kvh,
                                           int t, int d, float& kv_k, float& kv_v, bool want_v) {
  const int D = p.head_dim, BSZ = p.block_size;
  const int64_t row = (slot * p.kv_heads + kvh) * BSZ + t;
  if (state == HOT) {
    kv_k = __half2float(p.hot_k[row * D + d]);
    if (want_v) kv_v = __half2float(p.hot_v[row * D + d]);
  } else if (state == WARM) {
    if constexpr (WF == TIERKV_WARM_ABSMAX_I8) {
      const int8_t* wk = reinterpret_cast<const int8_t*>(p.warm_k);
      const int8_t* wv = reinterpret_cast<const int8_t*>(p.warm_v);
      const float sk = reinterpret_cast<const float*>(p.k_scale)[slot * p.kv_heads + kvh];
      kv_k = float(wk[row * D + d]) * sk;
      if (want_v) kv_v = float(wv[row * D + d]) * reinterpret_cast<const float*>(p.v_scale)[slot * p.kv_heads + kvh];
    } else {
      const uint8_t* wk = reinterpret_cast<const uint8_t*>(p.warm_k);
      const uint8_t* wv = reinterpret_cast<const uint8_t*>(p.warm_v);
      const __half* ks = reinterpret_cast<const __half*>(p.k_scale);
      const __half* kz = reinterpret_cast<const __half*>(p.k_zero);
      kv_k = (float(wk[row * D + d]) - __half2float(kz[row])) * __half2float(ks[row]);
      if (want_v) {
        const __half* vs = reinterpret_cast<const __half*>(p.v_scale);
        const __half* vz = reinterpret_cast<const __half*>(p.v_zero);
        kv_v = (float(wv[row * D + d]) - __half2float(vz[row])) * __half2float(vs[row]);
      }
    }
  } else {
    kv_k = 0.f;
    kv_v = 0.f;
  }
}

template <typename QT, int WF, bool COLD_ZERO>
__global__ __launch_bounds__(64) void decode_generic_kernel(DecodeParams p) {
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int lane = threadIdx.x;
  const int D = p.head_dim, BSZ = p.block_size;
  const int G = p.groups;
  const int kvh = h / G;
  const int nb = seq_blocks(p, b);
  const QT* qp = reinterpret_cast<const QT*>(p.q) + (int64_t(b) * p.num_heads + h) * D;
  constexpr int MAXR = 4;   // head_dim <= 256
  float acc[MAXR] = {0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;

  auto block_info = [&](int blk, int& st, int64_t& slot, int& len, bool& use) {
    const int64_t o = int64_t(b) * p.table_stride + blk;
    st = p.states[o];
    slot = p.table[o];
    len = min(max(p.lengths[o], 0), BSZ);
    use = len > 0;
    if (st == HOT || st == WARM) {
      const int64_t cap = (st == HOT) ? p.hot_slots : p.warm_slots;
      if (slot < 0 || slot >= cap) {
        if (use && lane == 0) atomicOr(p.ws_err, 1);
        use = false;
      }
    } else if (st == COLD) {
      use = use && COLD_ZERO;
    } else {
      if (lane == 0) atomicOr(p.ws_err, 2);
      use = false;
    }
  };

  auto logit_of = [&](int st, int64_t slot, int t) {
    float dot = 0.f;
    for (int d = 0; d < D; ++d) {
      float kk, vv;
      generic_kv<QT, WF>(p, st, slot, kvh, t, d, kk, vv, false);
      dot += kk * to_f32<QT>(qp[d]);
    }
    return dot * p.scaling;
  };

  for (int blk = 0; blk < nb; ++blk) {
    int st, len;
    int64_t slot;
    bool use;
    block_info(blk, st, slot, len, use);
    if (!use) continue;
    float x = -INFINITY;
    if (lane < len) x = (st == COLD) ? 0.f : logit_of(st, slot, lane);
    const float bm = wave_max(x);
    const float m_new = fmaxf(m, bm);
    const float alpha = (m == -INFINITY) ? 0.f : expf(m - m_new);
    const float pr = (lane < len) ? expf(x - m_new) : 0.f;
    l = l * alpha + wave_sum(pr);
#pragma unroll
    for (int r = 0; r < MAXR; ++r) acc[r] *= alpha;
    if (st != COLD) {
      for (int t = 0; t < len; ++t) {
        const float pt = __shfl(pr, t, 64);
#pragma unroll
        for (int r = 0; r < MAXR; ++r) {
          const int d = lane + 64 * r;
          if (d < D) {
            float kk, vv;
            generic_kv<QT, WF>(p, st, slot, kvh, t, d, kk, vv, true);
            acc[r] += pt * vv;
          }
        }
      }
    }
    m = m_new;
  }
#pragma unroll
  for (int r = 0; r < MAXR; ++r) {
    const int d = lane + 64 * r;
    if (d < D) {
      const float o = (l > 0.f) ? acc[r] / l : 0.f;
      reinterpret_cast<QT*>(p.out)[(int64_t(b) * p.num_heads + h) * D + d] = from_f32<QT>(o);
    }
  }
  if (p.score_sums) {
    float* sc = p.score_sums + (int64_t(b) * p.num_heads + h) * p.table_stride;
    for (int blk = 0; blk < int(p.table_stride); ++blk) {
      float v = 0.f;
      if (blk < nb && l > 0.f) {
        int st, len;
        int64_t slot;
        bool use;
        block_info(blk, st, slot, len, use);
        if (use) {
          const float x = (lane < len) ? ((st == COLD) ? 0.f : logit_of(st, slot, lane)) : -INFINITY;
          const float pr = (lane < len) ? expf(x - m) / l : 0.f;
          v = wave_sum(pr);
        }
      }
      if (lane == 0) sc[blk] = v;
    }
  }
}
// --------------------------------------------------------------------------
// Host side
// --------------------------------------------------------------------------

struct Plan {
  int nw;
  int splits;
};

static bool fast_path_ok(int block_size, int head_dim, int groups) {
  return block_size == FBS && (head_dim == 64 || head_dim == 128) && groups >= 1 && groups <= 16;
}

// Eight waves per workgroup (four for GQA groups above 8, to bound the LDS
// accumulators); enough splits to put about 2048 waves (two per SIMD) on the
// chip, but no more than one per 4*nw blocks of the row (a split costs a
// partial publish, an arrival and a merge, three dependent memory round
// trips, which only pays off when each split streams several tiles per
// wave), and enough that no split's list exceeds MAX_LIST.
static Plan plan_launch(int batch, int kv_heads, int num_blocks, int groups, int splits_hint) {
  Plan pl;
  pl.nw = groups <= 8 ? 8 : 4;
  const int64_t units = std::max<int64_t>(1, int64_t(batch) * kv_heads);
  int splits;
  if (splits_hint > 0) {
    splits = splits_hint;
  } else {
    const int64_t target_waves = 2048;
    splits = int(std::max<int64_t>(1, (target_waves + units * pl.nw - 1) / (units * pl.nw)));
    splits = std::min(splits, std::max(1, num_blocks / (4 * pl.nw)));
    // Rows under 12 tiles per wave stay whole: at 64 blocks one workgroup
    // per kv head took 6.96 us against 7.78 us for two splits (9.69 against
    // 12.71 us with score sums, which a split launch finalises in a second
    // launch); from 128 blocks on the splits above win.
    if (num_blocks < 12 * pl.nw) splits = 1;
  }
  // A split's list holds ceil(hot / splits) + ceil(warm / splits) entries,
  // at most ceil(num_blocks / splits) + 1: MAX_LIST - 1 blocks per split keep
  // the HOT (front) and WARM (back) halves of the list apart.
  splits = std::max(splits, (num_blocks + MAX_LIST - 2) / (MAX_LIST - 1));
  splits = std::min(splits, std::max(1, num_blocks));
  pl.splits = std::max(1, splits);
  return pl;
}

struct WsLayout {
  int64_t err, cnt, acc, ml, stage, total;
};

static WsLayout ws_layout(int batch, int num_heads, int kv_heads, int num_blocks, int block_size,
                          int head_dim, bool scores, int splits_hint) {
  WsLayout l{};
  const int groups = num_heads / std::max(kv_heads, 1);
  auto up = [](int64_t x) { return (x + 255) & ~int64_t(255); };
  l.err = 0;
  int64_t off = 256;
  if (fast_path_ok(block_size, head_dim, groups)) {
    const Plan pl = plan_launch(batch, kv_heads, num_blocks, groups, splits_hint);
    const int64_t units = int64_t(batch) * kv_heads;
    // The arrival counters come first and have the same place and size in
    // every layout, so a launch of any shape finds them zero.
    l.cnt = off;
    off = up(off + int64_t(MAX_SPLIT_UNITS) * 4);
    l.acc = off;
    if (pl.splits > 1) off = up(off + units * pl.splits * groups * head_dim * 4);
    l.ml = off;
    if (pl.splits > 1) off = up(off + units * pl.splits * groups * 2 * 4);
    l.stage = off;
    if (scores) off = up(off + int64_t(batch) * num_heads * num_blocks * 2 * 4);
  } else {
    l.cnt = l.acc = l.ml = l.stage = off;
  }
  l.total = off;
  return l;
}

template <int D, int WF, bool SC, bool CZ, typename QT, int NW>
static void launch_nw(const DecodeParams& p, bool long_rows, int grid, hipStream_t stream) {
  size_t shmem = size_t(NW) * p.groups * D * sizeof(float);
  if (SC && p.lds_stage == STAGE_LDS_BLOCK) shmem += size_t(p.groups) * p.num_blocks * 2 * sizeof(float);
  if (SC && p.lds_stage == STAGE_LDS_LIST) shmem += size_t(p.groups) * MAX_LIST * 2 * sizeof(float);
  const int32_t stride = int32_t(p.table_stride);
  const bool xcd_seq = p.splits == 1 && p.batch % 8 == 0;   // see tiered_decode_kernel
  const int32_t kvh_splits = int32_t(uint32_t(p.kv_heads) | (uint32_t(p.splits) << 16) |
                                     (p.deterministic ? 0x40000000u : 0u) | (xcd_seq ? 0x80000000u : 0u));
  if (long_rows)
    hipLaunchKernelGGL((tiered_decode_kernel<D, WF, SC, CZ, QT, NW, true>), dim3(grid), dim3(NW * 64), shmem, stream,
                       p.table, p.states, p.lengths, p.q, p.seq_nblocks, stride, p.num_blocks, kvh_splits,
                       p.split_magic, p);
  else
    hipLaunchKernelGGL((tiered_decode_kernel<D, WF, SC, CZ, QT, NW, false>), dim3(grid), dim3(NW * 64), shmem, stream,
                       p.table, p.states, p.lengths, p.q, p.seq_nblocks, stride, p.num_blocks, kvh_splits,
                       p.split_magic, p);
}

// Rows longer than one chunk of the workgroup's threads take the long-row
// list build.
template <int D, int WF, bool SC, bool CZ, typename QT>
static void launch_fast(const DecodeParams& p, int nw, int grid, hipStream_t stream) {
  const bool long_rows = p.num_blocks > nw * 64;
  if (nw == 8) launch_nw<D, WF, SC, CZ, QT, 8>(p, long_rows, grid, stream);
  else launch_nw<D, WF, SC, CZ, QT, 4>(p, long_rows, grid, stream);
}

template <int D, int WF, typename QT>
static void dispatch_sc_cz(const DecodeParams& p, bool sc, bool cz, int nw, int grid, hipStream_t stream) {
  if (sc) {
    if (cz) launch_fast<D, WF, true, true, QT>(p, nw, grid, stream);
    else launch_fast<D, WF, true, false, QT>(p, nw, grid, stream);
  } else {
    if (cz) launch_fast<D, WF, false, true, QT>(p, nw, grid, stream);
    else launch_fast<D, WF, false, false, QT>(p, nw, grid, stream);
  }
}

template <typename QT>
static void dispatch_fast(const DecodeParams& p, int wf, bool sc, bool cz, int nw, int grid, hipStream_t stream) {
  if (p.head_dim == 128) {
    if (wf == TIERKV_WARM_ABSMAX_I8) dispatch_sc_cz<128, TIERKV_WARM_ABSMAX_I8, QT>(p, sc, cz, nw, grid, stream);
    else dispatch_sc_cz<128, TIERKV_WARM_REF_U8, QT>(p, sc, cz, nw, grid, stream);
  } else {
    if (wf == TIERKV_WARM_ABSMAX_I8) dispatch_sc_cz<64, TIERKV_WARM_ABSMAX_I8, QT>(p, sc, cz, nw, grid, stream);
    else dispatch_sc_cz<64, TIERKV_WARM_REF_U8, QT>(p, sc, cz, nw, grid, stream);
  }
}

template <typename QT>
static void launch_generic(const DecodeParams& p, int wf, bool cz, hipStream_t stream) {
  dim3 grid(p.num_heads, p.batch);
  if (wf == TIERKV_WARM_ABSMAX_I8) {
    if (cz) hipLaunchKernelGGL((decode_generic_kernel<QT, TIERKV_WARM_ABSMAX_I8, true>), grid, dim3(64), 0, stream, p);
    else hipLaunchKernelGGL((decode_generic_kernel<QT, TIERKV_WARM_ABSMAX_I8, false>), grid, dim3(64), 0, stream, p);
  } else {
    if (cz) hipLaunchKernelGGL((decode_generic_kernel<QT, TIERKV_WARM_REF_U8, true>), grid, dim3(64), 0, stream, p);
    else hipLaunchKernelGGL((decode_generic_kernel<QT, TIERKV_WARM_REF_U8, false>), grid, dim3(64), 0, stream, p);
  }
}

}  // namespace tierkv

using namespace tierkv;

extern "C" int64_t tierkv_decode_workspace_bytes(int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                                 int32_t num_blocks, int32_t block_size, int32_t head_dim,
                                                 int32_t with_scores, int32_t splits_hint) {
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_blocks <= 0 || block_size <= 0 || head_dim <= 0)
    return -1;
  return ws_layout(batch, num_heads, num_kv_heads, num_blocks, block_size, head_dim, with_scores != 0,
                   hint_splits(splits_hint)).total;
}

// Every argument check of tierkv_decode_attention, before anything is
// launched (tierkv_decode_step runs it ahead of its token write, so a refused
// step changes nothing on the device).
int32_t tierkv::decode_check_args(
    const void* query, int32_t query_dtype, void* out, float* score_sums,
    const int32_t* block_table, const int32_t* block_states, const int32_t* block_lengths,
    int64_t table_stride, int32_t num_blocks,
    const void* hot_k, const void* hot_v, int64_t hot_slots,
    const void* warm_k, const void* warm_v, int64_t warm_slots,
    const void* k_scale, const void* k_zero, const void* v_scale, const void* v_zero,
    int32_t warm_format, int32_t cold_mode,
    int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t block_size, int32_t head_dim,
    int32_t splits_hint, void* workspace, int64_t workspace_bytes) {
  splits_hint = hint_splits(splits_hint);
  if (!query || !out || !block_table || !block_states || !block_lengths || !workspace)
    return fail(TIERKV_ERR_INVALID, "null tensor pointer");
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
    return fail(TIERKV_ERR_INVALID, "num_heads must be a positive multiple of num_kv_heads");
  if (num_blocks <= 0) return fail(TIERKV_ERR_INVALID, "num_blocks must be positive.");
  if (num_blocks > table_stride) return fail(TIERKV_ERR_INVALID, "num_blocks exceeds the provided block table length.");
  if (query_dtype != TIERKV_DTYPE_F16 && query_dtype != TIERKV_DTYPE_BF16)
    return fail(TIERKV_ERR_INVALID, "query dtype must be fp16 or bf16");
  if (warm_format != TIERKV_WARM_REF_U8 && warm_format != TIERKV_WARM_ABSMAX_I8)
    return fail(TIERKV_ERR_INVALID, "unknown warm format");
  if (cold_mode != TIERKV_COLD_ZERO_LOGIT && cold_mode != TIERKV_COLD_MASKED)
    return fail(TIERKV_ERR_INVALID, "unknown cold mode");
  if (block_size <= 0 || block_size > 64 || head_dim <= 0 || head_dim > 256)
    return fail(TIERKV_ERR_UNSUPPORTED, "block_size must be in [1, 64] and head_dim in [1, 256]");
  if (!hot_k || !hot_v || hot_slots <= 0) return fail(TIERKV_ERR_INVALID, "HOT pools are required");
  if (!warm_k || !warm_v || !k_scale || !v_scale || warm_slots <= 0)
    return fail(TIERKV_ERR_INVALID, "WARM pools and scales are required (pass 1-slot placeholders when empty)");
  if (warm_format == TIERKV_WARM_REF_U8 && (!k_zero || !v_zero))
    return fail(TIERKV_ERR_INVALID, "reference-format WARM pools need zero points");
  if (warm_format == TIERKV_WARM_ABSMAX_I8 && warm_slots * num_kv_heads * 4 > int64_t(0xffffffff))
    return fail(TIERKV_ERR_UNSUPPORTED, "absmax scale arrays of 4 GiB or more");
  if (int64_t(batch) * num_kv_heads > (int64_t(1) << 24))
    return fail(TIERKV_ERR_UNSUPPORTED, "batch * kv_heads too large");
  const bool scores = score_sums != nullptr;
  const WsLayout wl = ws_layout(batch, num_heads, num_kv_heads, num_blocks, block_size, head_dim, scores, splits_hint);
  if (workspace_bytes < wl.total) return fail(TIERKV_ERR_WORKSPACE, "workspace too small");
  const int groups = num_heads / num_kv_heads;
  if (fast_path_ok(block_size, head_dim, groups) && table_stride <= 0x7fffffff) {
    const bool aligned = aligned16(hot_k) && aligned16(hot_v) && aligned16(warm_k) && aligned16(warm_v) &&
                         aligned16(query);
    if (!aligned) return fail(TIERKV_ERR_INVALID, "query and pool base pointers must be 16-byte aligned");
    if (warm_format == TIERKV_WARM_REF_U8) {
      const uintptr_t m = reinterpret_cast<uintptr_t>(k_scale) | reinterpret_cast<uintptr_t>(k_zero) |
                          reinterpret_cast<uintptr_t>(v_scale) | reinterpret_cast<uintptr_t>(v_zero);
      if (m & 7u) return fail(TIERKV_ERR_INVALID, "reference-format scale/zero pools must be 8-byte aligned");
    }
    const Plan pl = plan_launch(batch, num_kv_heads, num_blocks, groups, splits_hint);
    if (pl.splits > 0x3fff || num_kv_heads > 0xffff)
      return fail(TIERKV_ERR_UNSUPPORTED, "more than 65535 kv heads or 16383 splits");
    int64_t seqs_per_chunk = batch;
    if (pl.splits > 1) {
      seqs_per_chunk = MAX_SPLIT_UNITS / num_kv_heads;
      if (seqs_per_chunk < 1) return fail(TIERKV_ERR_UNSUPPORTED, "too many kv heads for a split launch");
    }
    if (std::min<int64_t>(seqs_per_chunk, batch) * num_kv_heads * pl.splits > 0x7fffffff)
      return fail(TIERKV_ERR_UNSUPPORTED, "grid too large");
    if (scores && int64_t(batch) * num_heads > 0x7fffffff) return fail(TIERKV_ERR_UNSUPPORTED, "grid too large");
  }
  return TIERKV_OK;
}

extern "C" int32_t tierkv_decode_attention(
    const void* query, int32_t query_dtype, void* out, float* score_sums,
    const int32_t* block_table, const int32_t* block_states, const int32_t* block_lengths,
    int64_t table_stride, const int32_t* seq_num_blocks, int32_t num_blocks,
    const void* hot_k, const void* hot_v, int64_t hot_slots,
    const void* warm_k, const void* warm_v, int64_t warm_slots,
    const void* k_scale, const void* k_zero, const void* v_scale, const void* v_zero,
    int32_t warm_format, int32_t cold_mode,
    int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t block_size, int32_t head_dim,
    float scaling, int32_t splits_hint,
    void* workspace, int64_t workspace_bytes, void* stream_) {
  clear_error();
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  const bool det = hint_deterministic(splits_hint);
  splits_hint = hint_splits(splits_hint);
  const int32_t rc0 = decode_check_args(query, query_dtype, out, score_sums, block_table, block_states, block_lengths,
                                        table_stride, num_blocks, hot_k, hot_v, hot_slots, warm_k, warm_v, warm_slots,
                                        k_scale, k_zero, v_scale, v_zero, warm_format, cold_mode, batch, num_heads,
                                        num_kv_heads, block_size, head_dim, splits_hint, workspace, workspace_bytes);
  if (rc0 != TIERKV_OK) return rc0;
  const bool scores = score_sums != nullptr;
  const WsLayout wl = ws_layout(batch, num_heads, num_kv_heads, num_blocks, block_size, head_dim, scores, splits_hint);

  DecodeParams p{};
  p.q = query;
  p.out = out;
  p.table = block_table;
  p.states = block_states;
  p.lengths = block_lengths;
  p.table_stride = table_stride;
  p.seq_nblocks = seq_num_blocks;
  p.num_blocks = num_blocks;
  p.hot_k = reinterpret_cast<const __half*>(hot_k);
  p.hot_v = reinterpret_cast<const __half*>(hot_v);
  p.hot_slots = hot_slots;
  p.warm_k = warm_k;
  p.warm_v = warm_v;
  p.warm_slots = warm_slots;
  p.k_scale = k_scale;
  p.k_zero = k_zero;
  p.v_scale = v_scale;
  p.v_zero = v_zero;
  p.batch = batch;
  p.num_heads = num_heads;
  p.kv_heads = num_kv_heads;
  p.block_size = block_size;
  p.head_dim = head_dim;
  p.groups = num_heads / num_kv_heads;
  p.scaling = scaling;
  p.scale_log2 = scaling * LOG2E;
  char* ws = reinterpret_cast<char*>(workspace);
  p.ws_err = reinterpret_cast<int32_t*>(ws + wl.err);
  p.ws_cnt = reinterpret_cast<uint32_t*>(ws + wl.cnt);
  p.ws_acc = reinterpret_cast<float*>(ws + wl.acc);
  p.ws_ml = reinterpret_cast<float*>(ws + wl.ml);
  p.ws_stage = reinterpret_cast<float*>(ws + wl.stage);
  p.score_sums = score_sums;
  p.deterministic = det ? 1 : 0;
  const bool cz = cold_mode == TIERKV_COLD_ZERO_LOGIT;
  const bool bf16 = query_dtype == TIERKV_DTYPE_BF16;

  if (fast_path_ok(block_size, head_dim, p.groups) && table_stride <= 0x7fffffff) {
    // (alignment and launch limits: decode_check_args)
    const Plan pl = plan_launch(batch, num_kv_heads, num_blocks, p.groups, splits_hint);
    p.splits = pl.splits;
    p.split_magic = 0;
    // Unsplit score launches keep the per-block statistics in LDS (up to
    // MAX_LDS_STAGE bytes per workgroup) and finalise them in the workgroup;
    // split ones stage them in LDS by list position and copy them to the
    // workspace, where finalize_scores_kernel reads them.
    p.lds_stage = STAGE_GLOBAL;
    if (scores) {
      const int64_t pair = 2 * int64_t(sizeof(float));
      if (pl.splits == 1 && int64_t(p.groups) * num_blocks * pair <= MAX_LDS_STAGE) {
        p.lds_stage = STAGE_LDS_BLOCK;
      } else if (pl.splits > 1 && int64_t(p.groups) * MAX_LIST * pair <= MAX_LDS_STAGE) {
        p.lds_stage = STAGE_LDS_LIST;
      }
    }
    if (pl.splits > 1 && int64_t(num_blocks) * pl.splits < (int64_t(1) << 32))
      p.split_magic = uint32_t(((uint64_t(1) << 32) + uint64_t(pl.splits) - 1) / uint64_t(pl.splits));
    // Split launches go out in chunks of whole sequences, at most
    // MAX_SPLIT_UNITS units each (the size of the workspace's counter
    // region): each chunk is launched on offset pointers, so the kernel sees
    // a batch of its own.  Unsplit launches need no counters.
    const int64_t seqs_per_chunk = pl.splits > 1 ? MAX_SPLIT_UNITS / num_kv_heads : batch;
    const size_t qsz = bf16 ? sizeof(__hip_bfloat16) : sizeof(__half);
    for (int64_t b0 = 0; b0 < batch; b0 += seqs_per_chunk) {
      const int64_t nbat = std::min<int64_t>(seqs_per_chunk, batch - b0);
      DecodeParams pc = p;
      const int64_t u0 = b0 * num_kv_heads;
      pc.batch = int32_t(nbat);
      pc.q = reinterpret_cast<const char*>(p.q) + b0 * num_heads * head_dim * qsz;
      pc.out = reinterpret_cast<char*>(p.out) + b0 * num_heads * head_dim * qsz;
      pc.table = p.table + b0 * table_stride;
      pc.states = p.states + b0 * table_stride;
      pc.lengths = p.lengths + b0 * table_stride;
      if (p.seq_nblocks) pc.seq_nblocks = p.seq_nblocks + b0;
      if (p.score_sums) pc.score_sums = p.score_sums + b0 * num_heads * table_stride;
      pc.ws_stage = p.ws_stage + b0 * num_heads * int64_t(num_blocks) * 2;
      pc.ws_acc = p.ws_acc + u0 * pl.splits * p.groups * head_dim;
      pc.ws_ml = p.ws_ml + u0 * pl.splits * p.groups * 2;
      const int grid = int(nbat * num_kv_heads * pl.splits);
      if (bf16) dispatch_fast<__hip_bfloat16>(pc, warm_format, scores, cz, pl.nw, grid, stream);
      else dispatch_fast<__half>(pc, warm_format, scores, cz, pl.nw, grid, stream);
    }
    const int32_t rc = check_launch("tiered_decode_kernel");
    // Block stages are finalised inside the decode launch; list and
    // workspace stages by one workgroup per (sequence, q head) row.
    if (rc != TIERKV_OK || !scores || p.lds_stage == STAGE_LDS_BLOCK) return rc;
    const int parts = score_parts(p.groups, pl.nw);
    const int64_t rows = int64_t(batch) * num_heads;
    const size_t lds = num_blocks <= FIN_LDS_BLOCKS ? size_t(num_blocks) * sizeof(float2) : 0;
    const int32_t stride32 = int32_t(table_stride);
    if (cz)
      hipLaunchKernelGGL((finalize_scores_kernel<true>), dim3(unsigned(rows)), dim3(FIN_THREADS), lds, stream,
                         p.ws_stage, score_sums, seq_num_blocks, num_heads, num_blocks, stride32, parts);
    else
      hipLaunchKernelGGL((finalize_scores_kernel<false>), dim3(unsigned(rows)), dim3(FIN_THREADS), lds, stream,
                         p.ws_stage, score_sums, seq_num_blocks, num_heads, num_blocks, stride32, parts);
    return check_launch("finalize_scores_kernel");
  }
  p.splits = 1;
  if (bf16) launch_generic<__hip_bfloat16>(p, warm_format, cz, stream);
  else launch_generic<__half>(p, warm_format, cz, stream);
  return check_launch("decode_generic_kernel");
}

// --------------------------------------------------------------------------
// Allocation-free variant: the decode workspace is a file-scope device array
// (`scratch`), one copy per GPU, held until the process ends.
// --------------------------------------------------------------------------

namespace tierkv {
constexpr int64_t STATIC_SCRATCH_BYTES = int64_t(16) << 20;
constexpr int MAX_DEVICES = 64;
}  // namespace tierkv

static __device__ __align__(256) uint8_t scratch[tierkv::STATIC_SCRATCH_BYTES];

namespace tierkv {
namespace {

std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES] = {};   // device address of `scratch` on each GPU

__global__ void scratch_zero_kernel(uint4* p, int64_t n16) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += int64_t(gridDim.x) * blockDim.x)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// The current device's copy of `scratch`.  The first call on a device takes
// its address (host code never passes the array's name to a kernel), zeroes
// it on `stream` (refused under capture) and waits for the fill before the
// address is published, so a later call on any stream finds the array zero;
// later calls reuse the address.  The arrival counters and the error word
// must start at zero; every complete decode launch leaves the counters at
// zero again.
int32_t device_scratch(hipStream_t stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES)
    return fail(TIERKV_ERR_HIP, "tierkv_decode_attention_noalloc: no usable current device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    // The zero fill must run now, not at some later graph replay.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone)
      return fail(TIERKV_ERR_INVALID, "tierkv_decode_attention_noalloc: the first call on a device must not be "
                                      "under stream capture (it zeroes the device's scratch array)");
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(TIERKV_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    hipLaunchKernelGGL(scratch_zero_kernel, dim3(1024), dim3(256), 0, stream, reinterpret_cast<uint4*>(ptr),
                       STATIC_SCRATCH_BYTES / 16);
    const int32_t rc = check_launch("scratch_zero_kernel");
    if (rc != TIERKV_OK) return rc;
    const hipError_t se = hipStreamSynchronize(stream);
    if (se != hipSuccess)
      return fail(TIERKV_ERR_HIP, std::string("tierkv_decode_attention_noalloc: zeroing the scratch array: ") +
                                      hipGetErrorString(se));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return TIERKV_OK;
}

}  // namespace
}  // namespace tierkv

extern "C" int32_t tierkv_decode_attention_noalloc(
    const void* query, int32_t query_dtype, void* out, float* score_sums,
    const int32_t* block_table, const int32_t* block_states, const int32_t* block_lengths,
    int64_t table_stride, const int32_t* seq_num_blocks, int32_t num_blocks,
    const void* hot_k, const void* hot_v, int64_t hot_slots,
    const void* warm_k, const void* warm_v, int64_t warm_slots,
    const void* k_scale, const void* k_zero, const void* v_scale, const void* v_zero,
    int32_t warm_format, int32_t cold_mode,
    int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t block_size, int32_t head_dim,
    float scaling, int32_t splits_hint, void* stream_) {
  clear_error();
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  const int64_t need = tierkv_decode_workspace_bytes(batch, num_heads, num_kv_heads, num_blocks, block_size,
                                                     head_dim, score_sums != nullptr, splits_hint);
  if (need > STATIC_SCRATCH_BYTES)
    return fail(TIERKV_ERR_WORKSPACE, "tierkv_decode_attention_noalloc: this launch needs " + std::to_string(need) +
                                          " bytes of scratch; the allocation-free entry point holds " +
                                          std::to_string(STATIC_SCRATCH_BYTES) + " (use tierkv_decode_attention)");
  void* ws = nullptr;
  const int32_t rc = device_scratch(stream, &ws);
  if (rc != TIERKV_OK) return rc;
  return tierkv_decode_attention(query, query_dtype, out, score_sums, block_table, block_states, block_lengths,
                                 table_stride, seq_num_blocks, num_blocks, hot_k, hot_v, hot_slots, warm_k, warm_v,
                                 warm_slots, k_scale, k_zero, v_scale, v_zero, warm_format, cold_mode, batch,
                                 num_heads, num_kv_heads, block_size, head_dim, scaling, splits_hint, ws,
                                 STATIC_SCRATCH_BYTES, stream_);
}

extern "C" int32_t tierkv_decode_noalloc_error_word(int32_t clear, int32_t* word) {
  clear_error();
  if (!word) return fail(TIERKV_ERR_INVALID, "word must not be null");
  *word = 0;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES)
    return fail(TIERKV_ERR_HIP, "tierkv_decode_noalloc_error_word: no usable current device");
  void* ptr = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ptr = g_scratch_ptr[dev];
  }
  if (!ptr) return TIERKV_OK;   // no allocation-free launch on this device yet
  // The error word is the workspace layout's first word (offset 0).  Every
  // launch on the device, on any stream, completes before it is read.
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpy(word, ptr, sizeof(int32_t), hipMemcpyDeviceToHost);
  if (e == hipSuccess && clear && *word != 0) e = hipMemset(ptr, 0, sizeof(int32_t));
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess)
    return fail(TIERKV_ERR_HIP, std::string("tierkv_decode_noalloc_error_word: ") + hipGetErrorString(e));
  return TIERKV_OK;
}

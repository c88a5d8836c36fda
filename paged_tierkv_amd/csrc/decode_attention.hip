// Tiered paged decode attention for gfx950 (CDNA4).
//
// Replaces _tierkv_decode_attention_kernel (tierkv_triton.py:45-145) and the
// split/reduce pair (147-264) behind tierkv_decode_attention
// (tierkv_triton.py:272-465).
//
// Fast path (block_size 16, head_dim 64 or 128, GQA group <= 16):
//   * one workgroup = (sequence, kv head, split of logical blocks), 4 waves;
//     the whole GQA group is served by one pass over each K/V byte;
//   * the split's HOT/WARM blocks are compacted into an LDS list at start,
//     so COLD blocks cost no bytes and waves get a balanced round-robin share;
//   * one wave handles one 16-token block at a time with MFMA 16x16x16 f16:
//       S^T = K * Q^T   (A = K rows straight from HBM, B = Q^T, N = heads)
//       O^T += V^T * P^T (B = P^T is exactly S^T's accumulator layout)
//     WARM int8 codes are turned into fp16 in registers; absmax scales are
//     folded into the logits (s_k) and into P (s_v);
//   * online softmax in base 2 with wave-local state, merged across waves in
//     LDS and across splits in tierkv_decode_merge_kernel;
//   * the next block's tile is loaded while the current one is computed.
// Generic path (any block_size <= 64, head_dim <= 256, any group): one wave
// per (sequence, q head), the reference's two-pass structure.

#include "tierkv_common.h"

#include <algorithm>
#include <cfloat>
#include <cmath>

namespace tierkv {

constexpr int FBS = 16;          // tokens per block on the fast path
constexpr int NW = 4;            // waves per fast-path workgroup
constexpr int MAX_CHUNK = 256;   // logical blocks per split (LDS list capacity)
constexpr float PBOOST = 64.f;   // P is scaled by 2^6 before its fp16 cast
constexpr float LOG2E = 1.4426950408889634f;

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
  int32_t splits, blocks_per_split;
  float* ws_acc;      // [units][splits][G][D]
  float* ws_ml;       // [units][splits][G][2]
  float* ws_stage;    // [B][H][num_blocks][2]  (block max, block sum)
  int32_t* ws_err;
  float* score_sums;  // [B][H][table_stride] or null
  int32_t direct_out;
};

__device__ __forceinline__ int seq_blocks(const DecodeParams& p, int b) {
  int nb = p.num_blocks;
  if (p.seq_nblocks) nb = min(max(p.seq_nblocks[b], 0), p.num_blocks);
  return nb;
}

// --------------------------------------------------------------------------
// Fast path
// --------------------------------------------------------------------------

template <int D, int WF>
struct Tile {
  // HOT: lane's K slice (D/4 halves) and 4 tokens x D/16 halves of V.
  // WARM: the same bytes as 1-byte codes (first half of the arrays).
  uint32_t k[D / 8];
  uint32_t v[4][D / 32];
  float kmeta[2];        // REF_U8: this lane's token K scale / zero; ABSMAX: s_k
  float vmeta[4][2];     // REF_U8: per-token V scale / zero; ABSMAX: [0][0] = s_v
};

template <int D, int WF>
__device__ __forceinline__ void load_tile(const DecodeParams& p, int kvh, int4 e, int lane,
                                          Tile<D, WF>& t) {
  const int n = lane & 15;   // token row for K, dim group for V
  const int g = lane >> 4;   // dim quarter for K, token quad for V
  const int64_t slot = e.y;
  const int64_t tile0 = (slot * p.kv_heads + kvh) * FBS;   // first token row of the tile
  if (e.w == HOT) {
    const uint4* kp = reinterpret_cast<const uint4*>(p.hot_k + (tile0 + n) * D + g * (D / 4));
#pragma unroll
    for (int i = 0; i < D / 32; ++i) {
      uint4 x = kp[i];
      t.k[4 * i + 0] = x.x; t.k[4 * i + 1] = x.y; t.k[4 * i + 2] = x.z; t.k[4 * i + 3] = x.w;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const __half* vp = p.hot_v + (tile0 + 4 * g + j) * D + n * (D / 16);
      if constexpr (D == 128) {
        uint4 x = *reinterpret_cast<const uint4*>(vp);
        t.v[j][0] = x.x; t.v[j][1] = x.y; t.v[j][2] = x.z; t.v[j][3] = x.w;
      } else {
        uint2 x = *reinterpret_cast<const uint2*>(vp);
        t.v[j][0] = x.x; t.v[j][1] = x.y;
      }
    }
  } else {
    const uint8_t* wk = reinterpret_cast<const uint8_t*>(p.warm_k);
    const uint8_t* wv = reinterpret_cast<const uint8_t*>(p.warm_v);
    const uint4* kp = reinterpret_cast<const uint4*>(wk + (tile0 + n) * D + g * (D / 4));
#pragma unroll
    for (int i = 0; i < D / 64; ++i) {
      uint4 x = kp[i];
      t.k[4 * i + 0] = x.x; t.k[4 * i + 1] = x.y; t.k[4 * i + 2] = x.z; t.k[4 * i + 3] = x.w;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint8_t* vp = wv + (tile0 + 4 * g + j) * D + n * (D / 16);
      if constexpr (D == 128) {
        uint2 x = *reinterpret_cast<const uint2*>(vp);
        t.v[j][0] = x.x; t.v[j][1] = x.y;
      } else {
        t.v[j][0] = *reinterpret_cast<const uint32_t*>(vp);
      }
    }
    if constexpr (WF == TIERKV_WARM_ABSMAX_I8) {
      const float* ks = reinterpret_cast<const float*>(p.k_scale);
      const float* vs = reinterpret_cast<const float*>(p.v_scale);
      t.kmeta[0] = ks[slot * p.kv_heads + kvh];
      t.vmeta[0][0] = vs[slot * p.kv_heads + kvh];
    } else {
      const __half* ks = reinterpret_cast<const __half*>(p.k_scale);
      const __half* kz = reinterpret_cast<const __half*>(p.k_zero);
      const __half* vs = reinterpret_cast<const __half*>(p.v_scale);
      const __half* vz = reinterpret_cast<const __half*>(p.v_zero);
      t.kmeta[0] = __half2float(ks[tile0 + n]);
      t.kmeta[1] = __half2float(kz[tile0 + n]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        t.vmeta[j][0] = __half2float(vs[tile0 + 4 * g + j]);
        t.vmeta[j][1] = __half2float(vz[tile0 + 4 * g + j]);
      }
    }
  }
}

// K operand (A of S^T = K Q^T) for MFMA step s: dims g*D/4 + 4s .. +3 of
// token n.
template <int D, int WF>
__device__ __forceinline__ f16x4 k_operand(const Tile<D, WF>& t, int state, int s) {
  if (state == HOT) return as_f16x4(t.k[2 * s], t.k[2 * s + 1]);
  const uint32_t w = t.k[s];
  if constexpr (WF == TIERKV_WARM_ABSMAX_I8) {
    uint32_t lo, hi;
    i8x4_to_f16x4(w, lo, hi);
    return as_f16x4(lo, hi);
  } else {
    const float sc = t.kmeta[0], zp = t.kmeta[1];
    const float a0 = (float(w & 0xffu) - zp) * sc;
    const float a1 = (float((w >> 8) & 0xffu) - zp) * sc;
    const float a2 = (float((w >> 16) & 0xffu) - zp) * sc;
    const float a3 = (float(w >> 24) - zp) * sc;
    return as_f16x4(pack_f16x2(a0, a1), pack_f16x2(a2, a3));
  }
}

// V operand (A of O^T += V^T P^T) for step s: {V[4g+j][n*D/16 + s]}_{j=0..3}.
template <int D, int WF>
__device__ __forceinline__ f16x4 v_operand(const Tile<D, WF>& t, int state, int s) {
  if (state == HOT) {
    const int dw = s >> 1;
    if (s & 1) {
      return as_f16x4((t.v[0][dw] >> 16) | (t.v[1][dw] & 0xffff0000u),
                      (t.v[2][dw] >> 16) | (t.v[3][dw] & 0xffff0000u));
    }
    return as_f16x4((t.v[0][dw] & 0xffffu) | (t.v[1][dw] << 16),
                    (t.v[2][dw] & 0xffffu) | (t.v[3][dw] << 16));
  }
  const int dw = s >> 2, sh = (s & 3) * 8;
  const uint32_t b0 = (t.v[0][dw] >> sh) & 0xffu;
  const uint32_t b1 = (t.v[1][dw] >> sh) & 0xffu;
  const uint32_t b2 = (t.v[2][dw] >> sh) & 0xffu;
  const uint32_t b3 = (t.v[3][dw] >> sh) & 0xffu;
  if constexpr (WF == TIERKV_WARM_ABSMAX_I8) {
    uint32_t lo, hi;
    i8x4_to_f16x4(b0 | (b1 << 8) | (b2 << 16) | (b3 << 24), lo, hi);
    return as_f16x4(lo, hi);
  } else {
    const float v0 = (float(b0) - t.vmeta[0][1]) * t.vmeta[0][0];
    const float v1 = (float(b1) - t.vmeta[1][1]) * t.vmeta[1][0];
    const float v2 = (float(b2) - t.vmeta[2][1]) * t.vmeta[2][0];
    const float v3 = (float(b3) - t.vmeta[3][1]) * t.vmeta[3][0];
    return as_f16x4(pack_f16x2(v0, v1), pack_f16x2(v2, v3));
  }
}

template <int D, int WF, bool SCORES, bool COLD_ZERO, typename QT>
__global__ __launch_bounds__(NW * 64) void decode_split_kernel(DecodeParams p) {
  constexpr int DS = D / 16;   // MFMA steps per block for each product
  extern __shared__ float s_dyn[];               // [NW][G][D] partial accumulators
  __shared__ int4 s_list[MAX_CHUNK];             // (block, slot, len, state)
  __shared__ int s_wave_cnt[NW];
  __shared__ int s_cold_tokens;
  __shared__ float s_m[NW][16];
  __shared__ float s_l[NW][16];

  const int G = p.groups;
  const int splits = p.splits;
  const int wg = blockIdx.x;
  const int split = wg % splits;
  const int unit = wg / splits;
  const int b = unit / p.kv_heads;
  const int kvh = unit % p.kv_heads;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int nb = seq_blocks(p, b);
  const int c0 = split * p.blocks_per_split;
  const int c1 = min(c0 + p.blocks_per_split, nb);

  if (tid == 0) s_cold_tokens = 0;

  // ---- compact this split's resident (HOT/WARM) blocks into LDS ----------
  bool res = false;
  int4 ent = make_int4(0, 0, 0, COLD);
  const int idx = c0 + tid;
  if (tid < p.blocks_per_split && idx < c1) {
    const int64_t o = int64_t(b) * p.table_stride + idx;
    const int st = p.states[o];
    const int slot = p.table[o];
    const int len = min(max(p.lengths[o], 0), FBS);
    ent = make_int4(idx, slot, len, st);
    if (st == HOT || st == WARM) {
      const int64_t cap = (st == HOT) ? p.hot_slots : p.warm_slots;
      const bool slot_ok = slot >= 0 && slot < cap;
      if (!slot_ok && len > 0) atomicOr(p.ws_err, 1);
      res = slot_ok && len > 0;
      if (SCORES && !res) {
        for (int h = 0; h < G; ++h) {
          float* sp = p.ws_stage + ((int64_t(b) * p.num_heads + kvh * G + h) * p.num_blocks + idx) * 2;
          sp[0] = -INFINITY;
          sp[1] = 0.f;
        }
      }
    } else if (st != COLD) {
      atomicOr(p.ws_err, 2);
    }
  }
  __syncthreads();
  if (COLD_ZERO && ent.w == COLD && ent.z > 0) atomicAdd(&s_cold_tokens, ent.z);
  const uint64_t mask = __ballot(res);
  if (lane == 0) s_wave_cnt[w] = __popcll(mask);
  __syncthreads();
  int base = 0, nres = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    base += (i < w) ? s_wave_cnt[i] : 0;
    nres += s_wave_cnt[i];
  }
  if (res) s_list[base + __popcll(mask & ((1ull << lane) - 1ull))] = ent;
  __syncthreads();

  // ---- per-wave online softmax over the list ------------------------------
  const int n = lane & 15;
  const int g = lane >> 4;
  const bool head_ok = n < G;
  const int qh = kvh * G + n;

  uint32_t qv[D / 8];
  {
    const QT* qp = reinterpret_cast<const QT*>(p.q) + (int64_t(b) * p.num_heads + (head_ok ? qh : 0)) * D + g * (D / 4);
#pragma unroll
    for (int i = 0; i < D / 8; ++i) {
      float a = head_ok ? to_f32<QT>(qp[2 * i]) : 0.f;
      float c = head_ok ? to_f32<QT>(qp[2 * i + 1]) : 0.f;
      qv[i] = pack_f16x2(a, c);
    }
  }

  float m_run = -INFINITY;
  float l_run = 0.f;
  f32x4 acc[DS];
#pragma unroll
  for (int s = 0; s < DS; ++s) acc[s] = f32x4{0.f, 0.f, 0.f, 0.f};

  Tile<D, WF> cur, nxt;
  int k = w;
  if (k < nres) load_tile<D, WF>(p, kvh, s_list[k], lane, cur);
  while (k < nres) {
    const int4 e = s_list[k];
    const int kn = k + NW;
    if (kn < nres) load_tile<D, WF>(p, kvh, s_list[kn], lane, nxt);
    const int state = e.w;

    // S^T = K Q^T: lane holds S[head n][token 4g + j].
    f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      const f16x4 a = k_operand<D, WF>(cur, state, s);
      const f16x4 bq = as_f16x4(qv[2 * s], qv[2 * s + 1]);
      sacc = __builtin_amdgcn_mfma_f32_16x16x16f16(a, bq, sacc, 0, 0, 0);
    }
    float coef = p.scale_log2;
    float vcoef = PBOOST;
    if (state == WARM && WF == TIERKV_WARM_ABSMAX_I8) {
      coef *= cur.kmeta[0];
      vcoef *= cur.vmeta[0][0];
    }
    float x[4];
    float bm = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool valid = (4 * g + j) < e.z;
      x[j] = valid ? sacc[j] * coef : -INFINITY;
      bm = fmaxf(bm, x[j]);
    }
    bm = fmaxf(bm, shfl_xor_f(bm, 16));
    bm = fmaxf(bm, shfl_xor_f(bm, 32));
    float ex[4];
    float ls = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ex[j] = (x[j] == -INFINITY) ? 0.f : exp2f(x[j] - bm);
      ls += ex[j];
    }
    ls += shfl_xor_f(ls, 16);
    ls += shfl_xor_f(ls, 32);
    if (SCORES && g == 0 && head_ok) {
      float* sp = p.ws_stage + ((int64_t(b) * p.num_heads + qh) * p.num_blocks + e.x) * 2;
      sp[0] = bm;
      sp[1] = ls;
    }
    const float m_new = fmaxf(m_run, bm);
    const float alpha = (m_run == -INFINITY) ? 0.f : exp2f(m_run - m_new);
    const float beta = exp2f(bm - m_new);
    l_run = l_run * alpha + ls * beta;
    m_run = m_new;
    if (__any(alpha != 1.f)) {
#pragma unroll
      for (int s = 0; s < DS; ++s) acc[s] *= alpha;
    }
    const float pscale = beta * vcoef;
    const f16x4 pf = as_f16x4(pack_f16x2(ex[0] * pscale, ex[1] * pscale),
                              pack_f16x2(ex[2] * pscale, ex[3] * pscale));
    if (e.z < FBS) {
      // Partial block: zero the V rows past the length so stale tail data
      // (weighted by p == 0) cannot inject Inf/NaN through 0 * x.
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (4 * g + j >= e.z) {
#pragma unroll
          for (int i = 0; i < D / 32; ++i) cur.v[j][i] = 0u;
          cur.vmeta[j][0] = 0.f;
          cur.vmeta[j][1] = 0.f;
        }
      }
    }
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      const f16x4 av = v_operand<D, WF>(cur, state, s);
      acc[s] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, pf, acc[s], 0, 0, 0);
    }
    cur = nxt;
    k = kn;
  }

  // ---- merge the NW waves in LDS -------------------------------------------
  float* s_acc = s_dyn;   // [NW][G][D]
  if (head_ok) {
    if (g == 0) {
      s_m[w][n] = m_run;
      s_l[w][n] = l_run;
    }
    // acc[s][j] holds O[head n][(4g + j) * DS + s].
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int s = 0; s < DS; ++s) {
        s_acc[(w * G + n) * D + (4 * g + j) * DS + s] = acc[s][j];
      }
    }
  }
  __syncthreads();
  const float cold_tokens = COLD_ZERO ? float(s_cold_tokens) : 0.f;
  for (int i = tid; i < G * D; i += NW * 64) {
    const int h = i / D;
    const int d = i - h * D;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, s_m[ww][h]);
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      const float mw = s_m[ww][h];
      const float f = (mw == -INFINITY) ? 0.f : exp2f(mw - M);
      L += s_l[ww][h] * f;
      A += s_acc[(ww * G + h) * D + d] * f;
    }
    if (COLD_ZERO && cold_tokens > 0.f) {
      // COLD tokens: logit 0, V = 0 (tierkv_triton.py:92-102 masked loads).
      const float M2 = fmaxf(M, 0.f);
      const float f = (M == -INFINITY) ? 0.f : exp2f(M - M2);
      L = L * f + cold_tokens * exp2f(-M2);
      A *= f;
      M = M2;
    }
    if (p.direct_out) {
      const float o = (L > 0.f) ? A / (L * PBOOST) : 0.f;
      reinterpret_cast<QT*>(p.out)[(int64_t(b) * p.num_heads + kvh * G + h) * D + d] = from_f32<QT>(o);
    } else {
      const int64_t pi = (int64_t(unit) * splits + split) * G + h;
      p.ws_acc[pi * D + d] = A;
      if (d == 0) {
        p.ws_ml[pi * 2 + 0] = M;
        p.ws_ml[pi * 2 + 1] = L;
      }
    }
  }
}

// Merge of the splits (LSE combine, tierkv_triton.py:231-264) and the score
// finalisation: score = l_b * 2^(m_b - M) / L for HOT/WARM blocks,
// len * 2^(-M) / L for COLD blocks in zero-logit mode, 0 otherwise.
template <typename QT, bool COLD_ZERO>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeParams p) {
  __shared__ float s_M[64];
  __shared__ float s_L[64];
  const int unit = blockIdx.x;
  const int b = unit / p.kv_heads;
  const int kvh = unit % p.kv_heads;
  const int G = p.groups;
  const int D = p.head_dim;
  const int splits = p.splits;
  for (int h = threadIdx.x; h < G; h += blockDim.x) {
    float M = -INFINITY;
    for (int s = 0; s < splits; ++s) M = fmaxf(M, p.ws_ml[((int64_t(unit) * splits + s) * G + h) * 2]);
    float L = 0.f;
    for (int s = 0; s < splits; ++s) {
      const float* ml = p.ws_ml + ((int64_t(unit) * splits + s) * G + h) * 2;
      L += (ml[0] == -INFINITY) ? 0.f : ml[1] * exp2f(ml[0] - M);
    }
    s_M[h] = M;
    s_L[h] = L;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < G * D; i += blockDim.x) {
    const int h = i / D;
    const int d = i - h * D;
    const float M = s_M[h], L = s_L[h];
    float A = 0.f;
    for (int s = 0; s < splits; ++s) {
      const int64_t pi = (int64_t(unit) * splits + s) * G + h;
      const float ms = p.ws_ml[pi * 2];
      if (ms != -INFINITY) A += p.ws_acc[pi * D + d] * exp2f(ms - M);
    }
    const float o = (L > 0.f) ? A / (L * PBOOST) : 0.f;
    reinterpret_cast<QT*>(p.out)[(int64_t(b) * p.num_heads + kvh * G + h) * D + d] = from_f32<QT>(o);
  }
  if (p.score_sums) {
    const int nb = seq_blocks(p, b);
    const int stride = int(p.table_stride);
    for (int i = threadIdx.x; i < G * stride; i += blockDim.x) {
      const int h = i / stride;
      const int blk = i - h * stride;
      const int qh = kvh * G + h;
      float sc = 0.f;
      const float M = s_M[h], L = s_L[h];
      if (blk < nb && L > 0.f) {
        const int64_t o = int64_t(b) * p.table_stride + blk;
        const int st = p.states[o];
        if (st == COLD) {
          if (COLD_ZERO) sc = float(min(max(p.lengths[o], 0), p.block_size)) * exp2f(-M) / L;
        } else if (st == HOT || st == WARM) {
          const float* sp = p.ws_stage + ((int64_t(b) * p.num_heads + qh) * p.num_blocks + blk) * 2;
          if (sp[0] != -INFINITY) sc = sp[1] * exp2f(sp[0] - M) / L;
        }
      }
      p.score_sums[(int64_t(b) * p.num_heads + qh) * p.table_stride + blk] = sc;
    }
  }
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

struct SplitPlan {
  int splits;
  int blocks_per_split;
};

static SplitPlan plan_splits(int batch, int kv_heads, int num_blocks, int splits_hint) {
  const int units = std::max(1, batch * kv_heads);
  int splits;
  if (splits_hint > 0) {
    splits = splits_hint;
  } else {
    // Aim for about 4 workgroups per CU on 256 CUs.
    const int target = 1024;
    splits = std::max(1, (target + units - 1) / units);
    // Keep at least 8 logical blocks per split.
    splits = std::min(splits, std::max(1, num_blocks / 8));
  }
  int bps = (num_blocks + splits - 1) / splits;
  bps = std::max(1, std::min(bps, MAX_CHUNK));
  splits = (num_blocks + bps - 1) / bps;
  return {std::max(1, splits), bps};
}

static bool fast_path_ok(int block_size, int head_dim, int groups) {
  return block_size == FBS && (head_dim == 64 || head_dim == 128) && groups >= 1 && groups <= 16;
}

struct WsLayout {
  int64_t err, acc, ml, stage, total;
};

static WsLayout ws_layout(int batch, int num_heads, int kv_heads, int num_blocks, int block_size,
                          int head_dim, bool scores, int splits_hint) {
  WsLayout l{};
  const int groups = num_heads / std::max(kv_heads, 1);
  auto up = [](int64_t x) { return (x + 255) & ~int64_t(255); };
  l.err = 0;
  int64_t off = 256;
  if (fast_path_ok(block_size, head_dim, groups)) {
    const SplitPlan sp = plan_splits(batch, kv_heads, num_blocks, splits_hint);
    const int64_t units = int64_t(batch) * kv_heads;
    l.acc = off;
    off = up(off + units * sp.splits * groups * head_dim * 4);
    l.ml = off;
    off = up(off + units * sp.splits * groups * 2 * 4);
    l.stage = off;
    if (scores) off = up(off + int64_t(batch) * num_heads * num_blocks * 2 * 4);
  } else {
    l.acc = l.ml = l.stage = off;
  }
  l.total = off;
  return l;
}

template <int D, int WF, bool SC, bool CZ, typename QT>
static void launch_fast(const DecodeParams& p, int grid, hipStream_t stream) {
  const size_t shmem = size_t(NW) * p.groups * D * sizeof(float);
  hipLaunchKernelGGL((decode_split_kernel<D, WF, SC, CZ, QT>), dim3(grid), dim3(NW * 64), shmem, stream, p);
}

template <int D, int WF, typename QT>
static void dispatch_sc_cz(const DecodeParams& p, bool sc, bool cz, int grid, hipStream_t stream) {
  if (sc) {
    if (cz) launch_fast<D, WF, true, true, QT>(p, grid, stream);
    else launch_fast<D, WF, true, false, QT>(p, grid, stream);
  } else {
    if (cz) launch_fast<D, WF, false, true, QT>(p, grid, stream);
    else launch_fast<D, WF, false, false, QT>(p, grid, stream);
  }
}

template <typename QT>
static void dispatch_fast(const DecodeParams& p, int wf, bool sc, bool cz, int grid, hipStream_t stream) {
  if (p.head_dim == 128) {
    if (wf == TIERKV_WARM_ABSMAX_I8) dispatch_sc_cz<128, TIERKV_WARM_ABSMAX_I8, QT>(p, sc, cz, grid, stream);
    else dispatch_sc_cz<128, TIERKV_WARM_REF_U8, QT>(p, sc, cz, grid, stream);
  } else {
    if (wf == TIERKV_WARM_ABSMAX_I8) dispatch_sc_cz<64, TIERKV_WARM_ABSMAX_I8, QT>(p, sc, cz, grid, stream);
    else dispatch_sc_cz<64, TIERKV_WARM_REF_U8, QT>(p, sc, cz, grid, stream);
  }
}

template <typename QT>
static void launch_merge(const DecodeParams& p, bool cz, int units, hipStream_t stream) {
  if (cz) hipLaunchKernelGGL((decode_merge_kernel<QT, true>), dim3(units), dim3(256), 0, stream, p);
  else hipLaunchKernelGGL((decode_merge_kernel<QT, false>), dim3(units), dim3(256), 0, stream, p);
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
  return ws_layout(batch, num_heads, num_kv_heads, num_blocks, block_size, head_dim, with_scores != 0, splits_hint).total;
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
  const bool scores = score_sums != nullptr;
  const WsLayout wl = ws_layout(batch, num_heads, num_kv_heads, num_blocks, block_size, head_dim, scores, splits_hint);
  if (workspace_bytes < wl.total) return fail(TIERKV_ERR_WORKSPACE, "workspace too small");

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
  p.ws_acc = reinterpret_cast<float*>(ws + wl.acc);
  p.ws_ml = reinterpret_cast<float*>(ws + wl.ml);
  p.ws_stage = reinterpret_cast<float*>(ws + wl.stage);
  p.score_sums = score_sums;
  const bool cz = cold_mode == TIERKV_COLD_ZERO_LOGIT;
  const bool bf16 = query_dtype == TIERKV_DTYPE_BF16;

  if (fast_path_ok(block_size, head_dim, p.groups)) {
    const bool aligned = aligned16(hot_k) && aligned16(hot_v) && aligned16(warm_k) && aligned16(warm_v);
    if (!aligned) return fail(TIERKV_ERR_INVALID, "pool base pointers must be 16-byte aligned");
    const SplitPlan sp = plan_splits(batch, num_kv_heads, num_blocks, splits_hint);
    p.splits = sp.splits;
    p.blocks_per_split = sp.blocks_per_split;
    p.direct_out = (sp.splits == 1 && !scores) ? 1 : 0;
    const int units = batch * num_kv_heads;
    const int grid = units * sp.splits;
    if (bf16) dispatch_fast<__hip_bfloat16>(p, warm_format, scores, cz, grid, stream);
    else dispatch_fast<__half>(p, warm_format, scores, cz, grid, stream);
    int32_t rc = check_launch("decode_split_kernel");
    if (rc) return rc;
    if (!p.direct_out) {
      if (bf16) launch_merge<__hip_bfloat16>(p, cz, units, stream);
      else launch_merge<__half>(p, cz, units, stream);
      rc = check_launch("decode_merge_kernel");
      if (rc) return rc;
    }
    return TIERKV_OK;
  }
  p.splits = 1;
  p.blocks_per_split = num_blocks;
  if (bf16) launch_generic<__hip_bfloat16>(p, warm_format, cz, stream);
  else launch_generic<__half>(p, warm_format, cz, stream);
  return check_launch("decode_generic_kernel");
}

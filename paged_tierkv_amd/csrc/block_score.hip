// Block scores and tier labels on gfx950.
//
// * tierkv_block_mass_from_probs: per-block probability mass of fp32
//   probabilities [B, H, T] (the quantity of compute_block_scores,
//   tierkv_policy.py:1380-1389, and of block_scores_from_probability_sums,
//   1905-1912) with a fixed reduction order: per token a sequential sum over
//   heads, a pairwise xor-butterfly tree over the block's tokens, then / H
//   and / max(len, 1).
// * tierkv_block_scores_from_sums: block_scores_from_probability_sums on the
//   decode kernel's per-(head, block) sums.
// * tierkv_tier_labels: enforce_tiered_budget / enforce_budget
//   (tierkv_policy.py:1391-1477) for a batch of sequences, by counting ranks
//   (rank_i = #{j : s_j > s_i or (s_j == s_i and j < i)}), which is exactly
//   the order Python's stable descending sort produces.

#include "tierkv_common.h"

#include <algorithm>

namespace tierkv {

__global__ __launch_bounds__(256) void block_mass_kernel(const float* __restrict__ probs,
                                                         const int32_t* __restrict__ lengths,
                                                         float* __restrict__ out, int heads,
                                                         int tokens, int bs, int nblk) {
  const int b = blockIdx.y;
  const int tok = blockIdx.x * 256 + threadIdx.x;
  const bool in = tok < tokens;
  const int blk = in ? tok / bs : 0;
  const int pos = tok - blk * bs;
  const int len = !in ? 0 : (lengths ? min(max(lengths[int64_t(b) * nblk + blk], 0), bs) : bs);
  float acc = 0.f;
  if (in) {
    const float* p = probs + int64_t(b) * heads * tokens + tok;
#pragma unroll 8
    for (int h = 0; h < heads; ++h) acc += p[int64_t(h) * tokens];
    if (pos >= len) acc = 0.f;
  }
  for (int m = 1; m < bs; m <<= 1) acc += __shfl_xor(acc, m, 64);
  if (in && pos == 0) {
    const float s = __fdiv_rn(acc, float(heads));
    out[int64_t(b) * nblk + blk] = __fdiv_rn(s, float(max(len, 1)));
  }
}

// The same reduction for block_size a power of two >= 4 and 16-byte aligned
// probabilities, staged through LDS.  A workgroup of MASS_T threads covers
// MASS_Q four-token quads (256 tokens) of one sequence; per round of MASS_HC
// heads each of its MASS_T / MASS_Q head groups loads MASS_HPG head rows of
// the quads (16-byte loads, every thread's loads in flight together) into
// LDS, and the first wave sums every quad's heads in order from there.  The
// tokens of a quad are folded as (t0 + t1) + (t2 + t3) and the lanes of one
// block with an xor butterfly -- the same pairwise tree as block_mass_kernel,
// so the results are bit-identical.  Many small loads per workgroup from
// all of its waves reach HBM sooner than a few waves with long load queues.
constexpr int MASS_T = 512;                 // threads per workgroup
constexpr int MASS_Q = 64;                  // token quads per workgroup
constexpr int MASS_HC = 32;                 // heads staged per round
constexpr int MASS_HPG = MASS_HC / (MASS_T / MASS_Q);   // head rows per thread and round
static_assert(MASS_HPG * (MASS_T / MASS_Q) == MASS_HC, "head groups must tile a round");

__global__ __launch_bounds__(MASS_T) void block_mass_staged_kernel(const float* __restrict__ probs,
                                                                    const int32_t* __restrict__ lengths,
                                                                    float* __restrict__ out, int heads,
                                                                    int tokens, int bs, int nblk) {
  __shared__ f32x4 st[MASS_HC][MASS_Q];
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int q = tid % MASS_Q, g = tid / MASS_Q;
  const int quad0 = blockIdx.x * MASS_Q;
  const bool in_ld = (quad0 + q) * 4 < tokens;
  const f32x4* p = reinterpret_cast<const f32x4*>(probs + int64_t(b) * heads * tokens) + quad0 + q;
  const int64_t row = tokens / 4;
  float a[4] = {0.f, 0.f, 0.f, 0.f};
  for (int h0 = 0; h0 < heads; h0 += MASS_HC) {
    f32x4 v[MASS_HPG];
#pragma unroll
    for (int k = 0; k < MASS_HPG; ++k) {
      const int h = h0 + MASS_HPG * g + k;
      if (in_ld && h < heads) v[k] = __builtin_nontemporal_load(p + h * row);
    }
    if (h0 > 0) __syncthreads();   // the previous round's sums have read the stage
#pragma unroll
    for (int k = 0; k < MASS_HPG; ++k)
      if (in_ld && h0 + MASS_HPG * g + k < heads) st[MASS_HPG * g + k][q] = v[k];
    __syncthreads();
    if (tid < MASS_Q && in_ld) {
      const int hn = min(MASS_HC, heads - h0);
#pragma unroll 8
      for (int h = 0; h < hn; ++h) {
        const f32x4 x = st[h][tid];
#pragma unroll
        for (int e = 0; e < 4; ++e) a[e] += x[e];
      }
    }
  }
  if (tid >= MASS_Q) return;
  const int tok0 = (quad0 + tid) * 4;
  const bool in = tok0 < tokens;
  const int blk = in ? tok0 / bs : 0;
  const int pos = tok0 - blk * bs;
  const int len = !in ? 0 : (lengths ? min(max(lengths[int64_t(b) * nblk + blk], 0), bs) : bs);
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (pos + e >= len) a[e] = 0.f;
  float acc = (a[0] + a[1]) + (a[2] + a[3]);
  for (int m = 1; m < bs / 4; m <<= 1) acc += __shfl_xor(acc, m, 64);
  if (in && pos == 0) {
    const float s = __fdiv_rn(acc, float(heads));
    out[int64_t(b) * nblk + blk] = __fdiv_rn(s, float(max(len, 1)));
  }
}

__global__ __launch_bounds__(256) void scores_from_sums_kernel(const float* __restrict__ sums, int64_t sums_stride,
                                                               const int32_t* __restrict__ lengths, int64_t len_stride,
                                                               float* __restrict__ out, int heads, int nblk) {
  const int b = blockIdx.y;
  const int blk = blockIdx.x * 256 + threadIdx.x;
  if (blk >= nblk) return;
  float acc = 0.f;
  for (int h = 0; h < heads; ++h) acc += sums[(int64_t(b) * heads + h) * sums_stride + blk];
  const float s = __fdiv_rn(acc, float(heads));
  const int len = max(lengths[int64_t(b) * len_stride + blk], 1);
  out[int64_t(b) * nblk + blk] = __fdiv_rn(s, float(len));
}

constexpr int LABEL_MAX_BLOCKS = 8192;
constexpr int LABEL_WAVES = 4;                             // waves per workgroup
constexpr int LABEL_CAND = 4;                              // candidates per wave and pass
constexpr int LABEL_GROUP = LABEL_WAVES * LABEL_CAND;      // candidates per workgroup and pass
constexpr int LABEL_MAX_WG = 16;                           // workgroups per sequence

__device__ __forceinline__ int tier_label(int rank, bool ranked, int c, int mode, int n, int extra_hot, int warm,
                                          int demoted_state) {
  int desired;
  if (mode == 0) {
    desired = c;                       // hot_only: enforce_policy returns early
  } else if (!ranked) {
    desired = HOT;                     // reserved {0, n-1}; n <= 2 -> all HOT
  } else if (rank < extra_hot) {
    desired = HOT;
  } else if (mode == 2) {
    desired = (rank < extra_hot + warm) ? WARM : COLD;
  } else {
    desired = demoted_state;
  }
  if (mode != 0 && n > 2 && c == COLD && desired != COLD) desired = COLD;   // COLD is sticky
  return desired;
}

// Workgroups of LABEL_WAVES waves; min(ceil(n / LABEL_GROUP), LABEL_MAX_WG)
// of them per sequence.  A workgroup stages the sequence's scores in LDS
// once; each wave then takes LABEL_CAND candidates per pass and counts their
// ranks with the competitors in its lanes: per 64 competitors and candidate
// one 64-bit compare against the candidate's key (a wave-uniform value) and
// the population count of the resulting lane mask.  Spreading the
// candidates over the chip keeps each wave's count short.
__global__ __launch_bounds__(64 * LABEL_WAVES) void tier_labels_kernel(const float* __restrict__ scores,
                                                                       const int32_t* __restrict__ cur,
                                                                       int32_t* __restrict__ out, int64_t stride,
                                                                       int n, int hot_budget, int warm_budget,
                                                                       int mode, int demoted_state) {
  __shared__ float s_row[LABEL_MAX_BLOCKS];
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const bool rank_needed = mode != 0 && n > 2;
  if (rank_needed) {
    for (int i = tid; i < n; i += 64 * LABEL_WAVES) s_row[i] = scores[int64_t(b) * n + i];
    __syncthreads();
  }
  const int extra_hot = max(hot_budget - 2, 0);
  const int warm = max(warm_budget, 0);
  for (int c0 = (blockIdx.x * LABEL_WAVES + (tid >> 6)) * LABEL_CAND; c0 < n; c0 += gridDim.x * LABEL_GROUP) {
    const int ci = c0 + lane;
    const bool mine = lane < LABEL_CAND && ci < n;
    const int c = mine ? cur[int64_t(b) * stride + ci] : 0;
    int rank = 0;
    if (rank_needed) {
      // rank among the candidates j in [1, n - 1)
      const uint64_t kmine = label_key(s_row[min(ci, n - 1)], ci);
      int cnt[LABEL_CAND];
#pragma unroll
      for (int k = 0; k < LABEL_CAND; ++k) cnt[k] = 0;
      for (int j0 = 0; j0 < n; j0 += 256) {
        uint64_t kj[4];
        bool vj[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = j0 + 64 * e + lane;
          vj[e] = j >= 1 && j < n - 1;
          kj[e] = label_key(s_row[min(j, n - 1)], j);
        }
#pragma unroll
        for (int k = 0; k < LABEL_CAND; ++k) {
          const uint32_t lo = __builtin_amdgcn_readlane(uint32_t(kmine), k);
          const uint32_t hi = __builtin_amdgcn_readlane(uint32_t(kmine >> 32), k);
          const uint64_t kc = (uint64_t(hi) << 32) | lo;
#pragma unroll
          for (int e = 0; e < 4; ++e) cnt[k] += __popcll(__builtin_amdgcn_ballot_w64(vj[e] && kj[e] > kc));
        }
      }
#pragma unroll
      for (int k = 0; k < LABEL_CAND; ++k) rank = lane == k ? cnt[k] : rank;
    }
    if (mine) {
      const bool ranked = rank_needed && ci != 0 && ci != n - 1;
      out[int64_t(b) * stride + ci] = tier_label(rank, ranked, c, mode, n, extra_hot, warm, demoted_state);
    }
  }
}

}  // namespace tierkv

using namespace tierkv;

extern "C" int32_t tierkv_block_mass_from_probs(const float* probs, const int32_t* lengths, float* out,
                                                int32_t batch, int32_t num_heads, int32_t tokens,
                                                int32_t block_size, void* stream_) {
  clear_error();
  if (!probs || !out) return fail(TIERKV_ERR_INVALID, "null pointer");
  if (batch <= 0 || num_heads <= 0 || tokens <= 0) return fail(TIERKV_ERR_INVALID, "shape must be positive");
  if (block_size <= 0 || block_size > 64 || (block_size & (block_size - 1)) != 0)
    return fail(TIERKV_ERR_UNSUPPORTED, "block_size must be a power of two <= 64");
  if (tokens % block_size != 0) return fail(TIERKV_ERR_INVALID, "tokens must be a multiple of block_size");
  if (batch > 65535) return fail(TIERKV_ERR_UNSUPPORTED, "batch too large");
  const int nblk = tokens / block_size;
  if (block_size >= 4 && aligned16(probs)) {
    dim3 grid((tokens / 4 + MASS_Q - 1) / MASS_Q, batch);
    hipLaunchKernelGGL(block_mass_staged_kernel, grid, dim3(MASS_T), 0, reinterpret_cast<hipStream_t>(stream_),
                       probs, lengths, out, num_heads, tokens, block_size, nblk);
    return check_launch("block_mass_staged_kernel");
  }
  dim3 grid((tokens + 255) / 256, batch);
  hipLaunchKernelGGL(block_mass_kernel, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream_), probs,
                     lengths, out, num_heads, tokens, block_size, nblk);
  return check_launch("block_mass_kernel");
}

extern "C" int32_t tierkv_block_scores_from_sums(const float* score_sums, int64_t sums_stride,
                                                 const int32_t* lengths, int64_t len_stride, float* out,
                                                 int32_t batch, int32_t num_heads, int32_t num_blocks,
                                                 void* stream_) {
  clear_error();
  if (num_blocks == 0) return TIERKV_OK;
  if (!score_sums || !lengths || !out) return fail(TIERKV_ERR_INVALID, "null pointer");
  if (batch <= 0 || num_heads <= 0 || num_blocks < 0 || num_blocks > sums_stride || num_blocks > len_stride)
    return fail(TIERKV_ERR_INVALID, "bad shape");
  if (batch > 65535) return fail(TIERKV_ERR_UNSUPPORTED, "batch too large");
  dim3 grid((num_blocks + 255) / 256, batch);
  hipLaunchKernelGGL(scores_from_sums_kernel, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream_),
                     score_sums, sums_stride, lengths, len_stride, out, num_heads, num_blocks);
  return check_launch("scores_from_sums_kernel");
}

extern "C" int32_t tierkv_tier_labels(const float* scores, const int32_t* cur_states, int32_t* new_states,
                                      int64_t states_stride, int32_t batch, int32_t num_blocks,
                                      int32_t hot_budget, int32_t warm_budget, int32_t mode,
                                      int32_t demoted_state, void* stream_) {
  clear_error();
  if (num_blocks == 0) return TIERKV_OK;
  if (!scores || !cur_states || !new_states) return fail(TIERKV_ERR_INVALID, "null pointer");
  if (batch <= 0 || num_blocks < 0 || num_blocks > states_stride) return fail(TIERKV_ERR_INVALID, "bad shape");
  if (mode < 0 || mode > 2) return fail(TIERKV_ERR_INVALID, "mode must be 0 (hot_only), 1 (hot_warm) or 2 (hot_warm_cold)");
  if (mode == 1 && demoted_state != WARM && demoted_state != COLD)
    return fail(TIERKV_ERR_INVALID, "demoted_state must be WARM_STATE or COLD_STATE.");
  if (num_blocks > LABEL_MAX_BLOCKS) return fail(TIERKV_ERR_UNSUPPORTED, "too many blocks per sequence for the label kernel");
  if (batch > 65535) return fail(TIERKV_ERR_UNSUPPORTED, "batch too large");
  const dim3 grid(std::min((num_blocks + LABEL_GROUP - 1) / LABEL_GROUP, LABEL_MAX_WG), batch);
  hipLaunchKernelGGL(tier_labels_kernel, grid, dim3(64 * LABEL_WAVES), 0, reinterpret_cast<hipStream_t>(stream_), scores,
                     cur_states, new_states, states_stride, num_blocks, hot_budget, warm_budget, mode,
                     demoted_state);
  return check_launch("tier_labels_kernel");
}

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

// The same reduction with four consecutive tokens per thread (block_size a
// power of two >= 4, probs 16-byte aligned): each thread keeps up to 32
// 16-byte head-row loads in flight at once, sums every token over the heads
// in order, folds its four tokens as (t0 + t1) + (t2 + t3) and the lanes of
// one block with an xor butterfly -- the same pairwise tree as
// block_mass_kernel, so the results are bit-identical.
constexpr int MASS_T = 128;   // threads per workgroup (512 tokens)
constexpr int MASS_BATCH = 32;   // head rows loaded before they are summed

__global__ __launch_bounds__(MASS_T) void block_mass_vec4_kernel(const float* __restrict__ probs,
                                                                  const int32_t* __restrict__ lengths,
                                                                  float* __restrict__ out, int heads,
                                                                  int tokens, int bs, int nblk) {
  const int b = blockIdx.y;
  const int tok0 = (blockIdx.x * MASS_T + threadIdx.x) * 4;
  const bool in = tok0 < tokens;
  float a[4] = {0.f, 0.f, 0.f, 0.f};
  if (in) {
    const f32x4* p = reinterpret_cast<const f32x4*>(probs + int64_t(b) * heads * tokens + tok0);
    const int64_t row = tokens / 4;
    for (int h0 = 0; h0 < heads; h0 += MASS_BATCH) {
      f32x4 v[MASS_BATCH];
#pragma unroll
      for (int k = 0; k < MASS_BATCH; ++k)
        if (h0 + k < heads) v[k] = __builtin_nontemporal_load(p + (h0 + k) * row);
#pragma unroll
      for (int k = 0; k < MASS_BATCH; ++k) {
        if (h0 + k < heads) {
#pragma unroll
          for (int e = 0; e < 4; ++e) a[e] += v[k][e];
        }
      }
    }
  }
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
constexpr int LABEL_T = 1024;   // threads per sequence

// One workgroup per sequence.  Each candidate's rank is counted by `par`
// adjacent lanes (par = 1, 2, 4 or 8, as many as the 1024 threads allow),
// lane k of the group counting the candidates j = 1 + k, 1 + k + par, ...,
// so the lanes of a wave read consecutive keys; the partial counts are summed
// over the group with lane shuffles.
__global__ __launch_bounds__(LABEL_T) void tier_labels_kernel(const float* __restrict__ scores,
                                                              const int32_t* __restrict__ cur,
                                                              int32_t* __restrict__ out, int64_t stride,
                                                              int n, int hot_budget, int warm_budget,
                                                              int mode, int demoted_state) {
  __shared__ __align__(16) uint64_t key[LABEL_MAX_BLOCKS];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  for (int i = tid; i < n; i += LABEL_T) key[i] = label_key(scores[int64_t(b) * n + i], i);
  __syncthreads();
  const int extra_hot = max(hot_budget - 2, 0);
  const int warm = max(warm_budget, 0);
  int lpar = 0;
  while (lpar < 3 && (n << (lpar + 1)) <= LABEL_T) ++lpar;
  const int par = 1 << lpar;
  for (int t0 = 0; t0 < n * par; t0 += LABEL_T) {
    const int t = t0 + tid;
    const int i = t >> lpar;
    const int part = t & (par - 1);
    const bool ranked = i < n && mode != 0 && n > 2 && i != 0 && i != n - 1;
    int rank = 0;
    if (ranked) {
      // rank among the candidates j in [1, n - 1)
      const uint64_t ki = key[i];
      int j = 1 + part;
#pragma unroll 4
      for (; j < n - 1; j += par) rank += key[j] > ki ? 1 : 0;
    }
    for (int m = 1; m < par; m <<= 1) rank += __shfl_xor(rank, m, 64);
    if (i < n && part == 0) {
      const int c = cur[int64_t(b) * stride + i];
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
      out[int64_t(b) * stride + i] = desired;
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
    dim3 grid((tokens / 4 + MASS_T - 1) / MASS_T, batch);
    hipLaunchKernelGGL(block_mass_vec4_kernel, grid, dim3(MASS_T), 0, reinterpret_cast<hipStream_t>(stream_),
                       probs, lengths, out, num_heads, tokens, block_size, nblk);
    return check_launch("block_mass_vec4_kernel");
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
  hipLaunchKernelGGL(tier_labels_kernel, dim3(batch), dim3(LABEL_T), 0, reinterpret_cast<hipStream_t>(stream_), scores,
                     cur_states, new_states, states_stride, num_blocks, hot_budget, warm_budget, mode,
                     demoted_state);
  return check_launch("tier_labels_kernel");
}

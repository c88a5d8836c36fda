// Prefill block scores on gfx950 without materialising the attention
// probabilities.
//
// Replaces compute_block_scores on the prefill attention weights
// (tierkv_policy.py:1380-1389, called from modeling_llama.py:282-292): for one
// sequence, the mean causal-softmax probability of each key block over every
// query head and every query,
//
//   mass[blk] = sum_{h, q} sum_{t in blk} p[h, q, t] / (H * T) / len(blk),
//   p[h, q, t] = exp(s * q_h . k_t - lse[h, q])  for t <= q, 0 otherwise.
//
// The reference needs the eager attention's [B, H, T, T] probabilities; with
// SDPA it falls back to a sink + recency proxy (modeling_llama.py:294-302).
// Here the probabilities are recomputed on MFMA in two passes over K:
//   pass 1: per (head, query) log-sum-exp, each lane keeping a running
//           (max, sum) over the key columns it owns, merged across the 16
//           lanes of a row once at the end;
//   pass 2: p = exp2(x - lse2), summed per 16-key tile, a fixed-order wave
//           reduction per tile into LDS.
// Workgroup = (sequence, kv head, 64 queries), 4 waves of 16 queries, each
// wave serving the whole GQA group for its queries with one pass over each
// K tile.  Partial tile sums go to a workspace [B, H_kv, T/64, T/16] and a
// second kernel reduces them in a fixed order, so results are deterministic.
//
// MFMA 16x16x16: A = Q rows (lane l: query l%16), B = K^T (lane l: key l%16),
// both with the head dimension visited in the same permuted order
// d = 32*(s/2) + 8*(l/16) + 4*(s%2) + i, so each lane loads 16-byte runs; the
// accumulator holds S[q = 4*(l/16) + j][key = l%16].

#include "tierkv_common.h"

#include <cmath>

namespace tierkv {

constexpr int PS_WAVES = 4;
constexpr int PS_QB = 16 * PS_WAVES;       // queries per workgroup
constexpr int PS_MAX_TILES = 2048;         // 16-key tiles: T <= 32768
constexpr int PS_MAX_GROUP = 8;            // GQA group

typedef short bf16x4 __attribute__((ext_vector_type(4)));

template <typename T>
__device__ __forceinline__ f32x4 mfma16(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1, f32x4 c);

template <>
__device__ __forceinline__ f32x4 mfma16<__half>(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(as_f16x4(a0, a1), as_f16x4(b0, b1), c, 0, 0, 0);
}

template <>
__device__ __forceinline__ f32x4 mfma16<__hip_bfloat16>(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1,
                                                        f32x4 c) {
  union { uint32_t u[2]; bf16x4 v; } a, b;
  a.u[0] = a0;
  a.u[1] = a1;
  b.u[0] = b0;
  b.u[1] = b1;
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a.v, b.v, c, 0, 0, 0);
}

struct PrefillParams {
  const void* q;
  const void* k;
  int64_t qs_b, qs_h, qs_t;      // element strides of q [B, H, T, D]
  int64_t ks_b, ks_h, ks_t;      // element strides of k [B, H_kv, T, D]
  float* partial;                // [B, H_kv, nqb, ntiles]
  int32_t heads, kv_heads, tokens, nqb, ntiles;
  float scale_log2;
};

template <int D, typename T, int GMAX>
__global__ __launch_bounds__(64 * PS_WAVES) void prefill_block_mass_kernel(PrefillParams p) {
  constexpr int C = D / 32;          // 16-byte loads per row
  constexpr int DS = D / 16;         // MFMA steps
  __shared__ float s_blk[PS_WAVES][PS_MAX_TILES];
  const int qb = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  const int G = p.heads / p.kv_heads;
  const int Tn = p.tokens;
  const int q0 = qb * PS_QB + 16 * w;

  for (int i = threadIdx.x; i < PS_WAVES * PS_MAX_TILES; i += 64 * PS_WAVES) (&s_blk[0][0])[i] = 0.f;

  // Q A-operands: row q0 + n (clamped), head kvh * G + gh.
  uint32_t qa[GMAX][C * 4];
  {
    const int qrow = min(q0 + n, Tn - 1);
    const T* qbase = reinterpret_cast<const T*>(p.q) + b * p.qs_b + qrow * p.qs_t;
#pragma unroll
    for (int gh = 0; gh < GMAX; ++gh) {
      if (gh < G) {
        const T* row = qbase + int64_t(kvh * G + gh) * p.qs_h;
#pragma unroll
        for (int c = 0; c < C; ++c) {
          const uint4 v = *reinterpret_cast<const uint4*>(row + 32 * c + 8 * g);
          qa[gh][4 * c + 0] = v.x;
          qa[gh][4 * c + 1] = v.y;
          qa[gh][4 * c + 2] = v.z;
          qa[gh][4 * c + 3] = v.w;
        }
      } else {
#pragma unroll
        for (int c = 0; c < 4 * C; ++c) qa[gh][c] = 0u;
      }
    }
  }
  __syncthreads();
  // Waves whose queries all lie past the prompt add nothing (their LDS slots stay zero).
  const int last_tile = min((q0 + 15) >> 4, (Tn - 1) >> 4);
  const T* kbase = reinterpret_cast<const T*>(p.k) + b * p.ks_b + int64_t(kvh) * p.ks_h;

  auto load_k = [&](int kt, uint32_t* kb) {
    const int krow = min(kt * 16 + n, Tn - 1);
    const T* row = kbase + int64_t(krow) * p.ks_t;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const uint4 v = *reinterpret_cast<const uint4*>(row + 32 * c + 8 * g);
      kb[4 * c + 0] = v.x;
      kb[4 * c + 1] = v.y;
      kb[4 * c + 2] = v.z;
      kb[4 * c + 3] = v.w;
    }
  };
  auto scores = [&](const uint32_t* kb, int gh) {
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      const int c = s >> 1, h = s & 1;
      acc = mfma16<T>(qa[gh][4 * c + 2 * h], qa[gh][4 * c + 2 * h + 1], kb[4 * c + 2 * h], kb[4 * c + 2 * h + 1],
                      acc);
    }
    return acc;
  };

  // Pass 1: log-sum-exp (base 2) per (head, query row).
  float m[GMAX][4], l[GMAX][4];
#pragma unroll
  for (int gh = 0; gh < GMAX; ++gh)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      m[gh][j] = -INFINITY;
      l[gh][j] = 0.f;
    }
  if (q0 < Tn) {
    for (int kt = 0; kt <= last_tile; ++kt) {
      uint32_t kb[C * 4];
      load_k(kt, kb);
      const int key = kt * 16 + n;
#pragma unroll
      for (int gh = 0; gh < GMAX; ++gh) {
        if (gh >= G) continue;
        const f32x4 acc = scores(kb, gh);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int q = q0 + 4 * g + j;
          if (key <= q && q < Tn) {
            const float x = acc[j] * p.scale_log2;
            if (x > m[gh][j]) {
              l[gh][j] = l[gh][j] * exp2f(m[gh][j] - x) + 1.f;
              m[gh][j] = x;
            } else {
              l[gh][j] += exp2f(x - m[gh][j]);
            }
          }
        }
      }
    }
  }
  // Merge the 16 key-column owners of each row (lanes with equal l / 16).
  float lse[GMAX][4];
#pragma unroll
  for (int gh = 0; gh < GMAX; ++gh)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float mm = m[gh][j], ll = l[gh][j];
#pragma unroll
      for (int d = 1; d < 16; d <<= 1) {
        const float mo = shfl_xor_f(mm, d), lo = shfl_xor_f(ll, d);
        const float M = fmaxf(mm, mo);
        ll = (M == -INFINITY) ? 0.f : ll * exp2f(mm - M) + lo * exp2f(mo - M);
        mm = M;
      }
      lse[gh][j] = (ll > 0.f) ? mm + log2f(ll) : INFINITY;
    }

  // Pass 2: probability mass per 16-key tile.
  if (q0 < Tn) {
    for (int kt = 0; kt <= last_tile; ++kt) {
      uint32_t kb[C * 4];
      load_k(kt, kb);
      const int key = kt * 16 + n;
      float part = 0.f;
#pragma unroll
      for (int gh = 0; gh < GMAX; ++gh) {
        if (gh >= G) continue;
        const f32x4 acc = scores(kb, gh);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int q = q0 + 4 * g + j;
          if (key <= q && q < Tn) part += exp2f(acc[j] * p.scale_log2 - lse[gh][j]);
        }
      }
      part = wave_sum(part);
      if (lane == 0) s_blk[w][kt] = part;
    }
  }
  __syncthreads();
  float* out = p.partial + ((int64_t(b) * p.kv_heads + kvh) * p.nqb + qb) * p.ntiles;
  for (int kt = threadIdx.x; kt < p.ntiles; kt += 64 * PS_WAVES) {
    float acc = 0.f;
#pragma unroll
    for (int ww = 0; ww < PS_WAVES; ++ww) acc += s_blk[ww][kt];
    out[kt] = acc;
  }
}

// mass[b, blk] = sum over kv heads, query blocks and the block's tiles, in a
// fixed order, / (H * T) / len(blk).
__global__ __launch_bounds__(256) void prefill_mass_reduce_kernel(const float* partial, float* mass, int kv_heads,
                                                                   int nqb, int ntiles, int heads, int tokens,
                                                                   int block_size, int nblk) {
  const int b = blockIdx.y;
  const int blk = blockIdx.x * 256 + threadIdx.x;
  if (blk >= nblk) return;
  const int tpb = block_size / 16;
  float acc = 0.f;
  for (int h = 0; h < kv_heads; ++h)
    for (int qb = 0; qb < nqb; ++qb) {
      const float* row = partial + ((int64_t(b) * kv_heads + h) * nqb + qb) * ntiles;
      for (int t = blk * tpb; t < min((blk + 1) * tpb, ntiles); ++t) acc += row[t];
    }
  const int len = min(block_size, tokens - blk * block_size);
  mass[int64_t(b) * nblk + blk] = acc / (float(heads) * float(tokens)) / float(max(len, 1));
}

template <int D, typename T>
static hipError_t launch_prefill(const PrefillParams& p, int batch, int G, hipStream_t stream) {
  const dim3 grid(p.nqb, p.kv_heads, batch);
  if (G <= 4)
    hipLaunchKernelGGL((prefill_block_mass_kernel<D, T, 4>), grid, dim3(64 * PS_WAVES), 0, stream, p);
  else
    hipLaunchKernelGGL((prefill_block_mass_kernel<D, T, PS_MAX_GROUP>), grid, dim3(64 * PS_WAVES), 0, stream, p);
  return hipGetLastError();
}

}  // namespace tierkv

using namespace tierkv;

extern "C" int64_t tierkv_prefill_block_mass_workspace_bytes(int32_t batch, int32_t num_kv_heads, int32_t tokens) {
  if (batch <= 0 || num_kv_heads <= 0 || tokens <= 0) return -1;
  const int64_t nqb = (tokens + PS_QB - 1) / PS_QB;
  const int64_t ntiles = (tokens + 15) / 16;
  return int64_t(batch) * num_kv_heads * nqb * ntiles * 4;
}

extern "C" int32_t tierkv_prefill_block_mass(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_t,
    const void* k, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_t, int32_t dtype,
    float* mass, int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t tokens, int32_t head_dim,
    int32_t block_size, float scaling, void* workspace, int64_t workspace_bytes, void* stream_) {
  clear_error();
  if (!q || !k || !mass || !workspace) return fail(TIERKV_ERR_INVALID, "null pointer");
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || tokens <= 0)
    return fail(TIERKV_ERR_INVALID, "empty prefill");
  if (num_heads % num_kv_heads != 0) return fail(TIERKV_ERR_INVALID, "num_heads must be a multiple of num_kv_heads");
  const int G = num_heads / num_kv_heads;
  if (G > PS_MAX_GROUP) return fail(TIERKV_ERR_UNSUPPORTED, "GQA group above 8");
  if (head_dim != 64 && head_dim != 128) return fail(TIERKV_ERR_UNSUPPORTED, "head_dim must be 64 or 128");
  if (block_size <= 0 || block_size % 16 != 0) return fail(TIERKV_ERR_UNSUPPORTED, "block_size must be a multiple of 16");
  if ((tokens + 15) / 16 > PS_MAX_TILES) return fail(TIERKV_ERR_UNSUPPORTED, "prompts above 32768 tokens");
  if (dtype != TIERKV_DTYPE_F16 && dtype != TIERKV_DTYPE_BF16) return fail(TIERKV_ERR_INVALID, "unknown dtype");
  // Every row load is 16 bytes at element offsets that are multiples of 8.
  const int64_t strides[6] = {q_stride_b, q_stride_h, q_stride_t, k_stride_b, k_stride_h, k_stride_t};
  for (int64_t s : strides)
    if (s % 8 != 0) return fail(TIERKV_ERR_INVALID, "q/k strides must be multiples of 8 elements");
  if (!aligned16(q) || !aligned16(k)) return fail(TIERKV_ERR_INVALID, "q and k must be 16-byte aligned");
  const int64_t need = tierkv_prefill_block_mass_workspace_bytes(batch, num_kv_heads, tokens);
  if (workspace_bytes < need) return fail(TIERKV_ERR_INVALID, "workspace too small");
  PrefillParams p{};
  p.q = q;
  p.k = k;
  p.qs_b = q_stride_b;
  p.qs_h = q_stride_h;
  p.qs_t = q_stride_t;
  p.ks_b = k_stride_b;
  p.ks_h = k_stride_h;
  p.ks_t = k_stride_t;
  p.partial = reinterpret_cast<float*>(workspace);
  p.heads = num_heads;
  p.kv_heads = num_kv_heads;
  p.tokens = tokens;
  p.nqb = (tokens + PS_QB - 1) / PS_QB;
  p.ntiles = (tokens + 15) / 16;
  p.scale_log2 = scaling * 1.4426950408889634f;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  hipError_t e;
  if (dtype == TIERKV_DTYPE_F16)
    e = head_dim == 128 ? launch_prefill<128, __half>(p, batch, G, stream) : launch_prefill<64, __half>(p, batch, G, stream);
  else
    e = head_dim == 128 ? launch_prefill<128, __hip_bfloat16>(p, batch, G, stream)
                        : launch_prefill<64, __hip_bfloat16>(p, batch, G, stream);
  if (e != hipSuccess) return fail(TIERKV_ERR_HIP, std::string("prefill_block_mass_kernel: ") + hipGetErrorString(e));
  const int nblk = (tokens + block_size - 1) / block_size;
  hipLaunchKernelGGL(prefill_mass_reduce_kernel, dim3((nblk + 255) / 256, batch), dim3(256), 0, stream, p.partial,
                     mass, num_kv_heads, p.nqb, p.ntiles, num_heads, tokens, block_size, nblk);
  return check_launch("prefill_mass_reduce_kernel");
}

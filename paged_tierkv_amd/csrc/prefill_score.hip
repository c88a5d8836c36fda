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
//           (max, sum) over the keys it owns; the maximum is re-based only
//           when a logit exceeds it by more than PS_LAZY (log2 units), and
//           the four key-row owners of a query are merged once at the end;
//   pass 2: p = exp2(x - lse2), summed per 16-key tile in the lane, then one
//           fixed-order wave reduction per tile into LDS.
// Workgroup = (sequence, kv head, 64 queries), 4 waves of 16 queries, each
// wave serving the whole GQA group for its queries with one pass over each
// K tile; the next K tile is loaded while the current one is processed.
// Partial tile sums go to a workspace [B, H_kv, T/64, T/16] and a second
// kernel reduces them in a fixed order, so results are deterministic.
//
// MFMA 16x16x32 (gfx950): A = K tile (lane l: key l%16), B = Q^T (lane l:
// query l%16), both with the head dimension visited in the same order
// d = 32*s + 8*(l/16) + i (16-byte loads); the accumulator holds
// S^T[key = 4*(l/16) + j][query = l%16], so a lane's four logits belong to
// one query and the per-query sums need no shuffles until the end.

#include "tierkv_common.h"

#include <cmath>
#include <type_traits>

namespace tierkv {

constexpr int PS_WAVES = 4;
constexpr int PS_QB = 16 * PS_WAVES;       // queries per workgroup
constexpr int PS_MAX_TILES = 2048;         // 16-key tiles: T <= 32768
constexpr int PS_MAX_GROUP = 8;            // GQA group

constexpr float PS_LAZY = 8.f;             // log2 headroom of the running maximum
constexpr float PS_FLOOR = -1e30f;         // initial running maximum (finite)

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <typename T>
__device__ __forceinline__ f32x4 mfma32(const uint4& a, const uint4& b, f32x4 c);

template <>
__device__ __forceinline__ f32x4 mfma32<__half>(const uint4& a, const uint4& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                0);
}

template <>
__device__ __forceinline__ f32x4 mfma32<__hip_bfloat16>(const uint4& a, const uint4& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}

struct PrefillParams {
  const void* q;
  const void* k;
  int64_t qs_b, qs_h, qs_t;      // element strides of q [B, H, T, D]
  int64_t ks_b, ks_h, ks_t;      // element strides of k [B, H_kv, T, D]
  float* partial;                // [B, H_kv, nqb, PS_WAVES, ntiles]
  int32_t heads, kv_heads, tokens, nqb, ntiles, batch;
  float scale_log2;
};

// EXACT: the GQA group is exactly GMAX (no per-head guards).
template <int D, typename T, int GMAX, bool EXACT>
__global__ __launch_bounds__(64 * PS_WAVES) void prefill_block_mass_kernel(PrefillParams p) {
  constexpr int KS = D / 32;         // MFMA k-steps (one 16-byte load each)
  constexpr int RC = D / 8;          // 16-byte chunks per K row
  constexpr int RP = RC + 1;         // LDS row pitch in chunks (one pad chunk against bank conflicts)
  // The workgroup's current and next K tile, staged once for its four waves.
  __shared__ uint4 s_k[2][16 * RP];
  // Workgroup -> (query block, kv head, sequence).  The hardware deals
  // consecutive workgroups to the 8 XCDs in turn; when the (sequence, kv
  // head) pairs come in multiples of 8, all query blocks of one pair go to
  // the same XCD, so its K stays in that XCD's L2.  Query blocks run in
  // reverse: the longest causal rows are dispatched first.
  const int wg = int(blockIdx.x);
  const int npairs = p.kv_heads * p.batch;
  int pair, qi;
  if ((npairs & 7) == 0) {
    const int slot = wg >> 3;
    pair = (slot / p.nqb) * 8 + (wg & 7);
    qi = slot % p.nqb;
  } else {
    pair = wg / p.nqb;
    qi = wg % p.nqb;
  }
  const int qb = p.nqb - 1 - qi, kvh = pair % p.kv_heads, b = pair / p.kv_heads;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  const int G = EXACT ? GMAX : p.heads / p.kv_heads;
  const int Tn = p.tokens;
  const int q0 = qb * PS_QB + 16 * w;

  // Q^T B-operands: query q0 + n (clamped), head kvh * G + gh.
  uint4 qv[GMAX][KS];
  {
    const int qrow = min(q0 + n, Tn - 1);
    const T* qbase = reinterpret_cast<const T*>(p.q) + b * p.qs_b + qrow * p.qs_t;
#pragma unroll
    for (int gh = 0; gh < GMAX; ++gh) {
      if (EXACT || gh < G) {
        const T* row = qbase + int64_t(kvh * G + gh) * p.qs_h;
#pragma unroll
        for (int s = 0; s < KS; ++s) qv[gh][s] = *reinterpret_cast<const uint4*>(row + 32 * s + 8 * g);
      } else {
#pragma unroll
        for (int s = 0; s < KS; ++s) qv[gh][s] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
  }
  // Waves whose queries all lie past the prompt compute nothing (the reduce
  // kernel skips their tiles).
  const int last_tile = min((q0 + 15) >> 4, (Tn - 1) >> 4);
  const int wg_last = min((qb * PS_QB + PS_QB - 1) >> 4, (Tn - 1) >> 4);
  const int diag = q0 >> 4;                  // the one tile that needs the causal mask
  const bool row_ok = q0 + n < Tn;
  const bool rows_ok = q0 + 15 < Tn;        // every query of the wave lies in the prompt
  const bool active = q0 < Tn;
  const int kend = rows_ok ? last_tile : 0;  // tiles [0, kend) need no mask
  const T* kbase = reinterpret_cast<const T*>(p.k) + b * p.ks_b + int64_t(kvh) * p.ks_h;
  const float sl = p.scale_log2;
  // Cooperative K staging: thread t moves 16 bytes, chunk t % RC of row t / RC.
  const int lrow = threadIdx.x / RC, lchunk = threadIdx.x % RC;
  constexpr int LOADERS = 16 * RC;           // 256 (D = 128) or 128 (D = 64) threads
  auto fetch_k = [&](int kt) -> uint4 {
    const int krow = min(kt * 16 + lrow, Tn - 1);
    return *reinterpret_cast<const uint4*>(kbase + int64_t(krow) * p.ks_t + 8 * lchunk);
  };

  // The four raw logits q . k of keys kt*16 + 4g + j for this lane's query;
  // MASK: -inf where masked (past the query, or a query past the prompt).
  auto logits = [&](auto MASK, const uint4* sk, int gh, int kt, float* x) {
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) acc = mfma32<T>(sk[n * RP + 4 * s + g], qv[gh][s], acc);
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = acc[j];
    if constexpr (decltype(MASK)::value) {
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = (row_ok && (kt != diag || 4 * g + j <= n)) ? x[j] : -INFINITY;
    }
  };
  using NoMask = std::integral_constant<bool, false>;
  using Mask = std::integral_constant<bool, true>;

  // Both passes walk the workgroup's tiles [0, wg_last]: each tile is loaded
  // from global memory one tile ahead, written into the other LDS buffer
  // after the current one is processed, with one barrier per tile.  A wave
  // processes the tiles up to its own last one (below the diagonal without
  // masks, the diagonal tile with them).
  auto walk = [&](auto&& tile) {
    uint4 nxt = make_uint4(0u, 0u, 0u, 0u);
    if (threadIdx.x < LOADERS) s_k[0][lrow * RP + lchunk] = fetch_k(0);
    __syncthreads();
    for (int kt = 0; kt <= wg_last; ++kt) {
      const int cur = kt & 1;
      if (kt < wg_last && threadIdx.x < LOADERS) nxt = fetch_k(kt + 1);
      if (active && kt <= last_tile) {
        if (kt < kend) tile(NoMask{}, kt, s_k[cur]);
        else tile(Mask{}, kt, s_k[cur]);
      }
      if (kt < wg_last && threadIdx.x < LOADERS) s_k[cur ^ 1][lrow * RP + lchunk] = nxt;
      __syncthreads();
    }
  };

  // Pass 1: log-sum-exp (base 2) per (head, query), lazily re-based.  The
  // running maximum starts at a finite floor, so a lane that has seen only
  // masked keys (-inf) adds exp2(-inf) = 0 rather than exp2(-inf + inf).
  float m[GMAX], l[GMAX];
#pragma unroll
  for (int gh = 0; gh < GMAX; ++gh) {
    m[gh] = PS_FLOOR;
    l[gh] = 0.f;
  }
  walk([&](auto MASK, int kt, const uint4* sk) {
#pragma unroll
    for (int gh = 0; gh < GMAX; ++gh) {
      if (!EXACT && gh >= G) continue;
      float x[4];
      logits(MASK, sk, gh, kt, x);
      const float tm = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])) * sl;
      // Re-base where a logit exceeds the running maximum by more than
      // PS_LAZY (a wave-uniform test; rare after the first tiles).
      if (__any(tm > m[gh] + PS_LAZY)) {
        const bool up = tm > m[gh] + PS_LAZY;
        l[gh] *= up ? __builtin_amdgcn_exp2f(m[gh] - tm) : 1.f;
        m[gh] = up ? tm : m[gh];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) l[gh] += __builtin_amdgcn_exp2f(fmaf(x[j], sl, -m[gh]));
    }
  });
  // Merge the four key-row owners of each query (lanes n, n+16, n+32, n+48).
  float lse[GMAX];
#pragma unroll
  for (int gh = 0; gh < GMAX; ++gh) {
    float mm = m[gh], ll = l[gh];
#pragma unroll
    for (int d = 16; d < 64; d <<= 1) {
      const float mo = shfl_xor_f(mm, d), lo = shfl_xor_f(ll, d);
      const float M = fmaxf(mm, mo);
      ll = ll * __builtin_amdgcn_exp2f(mm - M) + lo * __builtin_amdgcn_exp2f(mo - M);
      mm = M;
    }
    lse[gh] = (ll > 0.f) ? mm + log2f(ll) : INFINITY;
  }

  // Pass 2: probability mass per 16-key tile, one value per (wave, tile)
  // into the workspace.
  float* out = p.partial + (((int64_t(b) * p.kv_heads + kvh) * p.nqb + qb) * PS_WAVES + w) * p.ntiles;
  walk([&](auto MASK, int kt, const uint4* sk) {
    float part = 0.f;
#pragma unroll
    for (int gh = 0; gh < GMAX; ++gh) {
      if (!EXACT && gh >= G) continue;
      float x[4];
      logits(MASK, sk, gh, kt, x);
#pragma unroll
      for (int j = 0; j < 4; ++j) part += __builtin_amdgcn_exp2f(fmaf(x[j], sl, -lse[gh]));
    }
    part = wave_sum_dpp(part);
    if (lane == 0) out[kt] = part;
  });
}

// mass[b, blk] = sum over kv heads, query blocks, waves and the block's
// tiles of the per-(wave, tile) sums, in a fixed order (lane i of the
// block's wave takes elements i, i + 64, ... of the (kv head, query block,
// wave, tile) enumeration, then a fixed DPP reduction), / (H * T) / len(blk).
// A wave's sums exist for its tiles up to its diagonal (tile <= 4 * query
// block + wave) and only if its first query lies in the prompt.  One wave per
// (sequence, block).
__global__ __launch_bounds__(64) void prefill_mass_reduce_kernel(const float* partial, float* mass, int kv_heads,
                                                                  int nqb, int ntiles, int heads, int tokens,
                                                                  int block_size, int nblk) {
  const int b = blockIdx.y;
  const int blk = blockIdx.x;
  const int lane = threadIdx.x;
  const int tpb = block_size / 16;
  const int t0 = blk * tpb;
  const int tn = min(tpb, ntiles - t0);
  const int total = kv_heads * nqb * PS_WAVES * tn;
  float acc = 0.f;
  for (int e = lane; e < total; e += 64) {
    const int t = t0 + e % tn;
    const int hqw = e / tn;                     // (h * nqb + qb) * PS_WAVES + w
    const int w = hqw % PS_WAVES;
    const int qb = (hqw / PS_WAVES) % nqb;
    if (t <= PS_WAVES * qb + w && qb * PS_QB + 16 * w < tokens)
      acc += partial[(int64_t(b) * kv_heads * nqb * PS_WAVES + hqw) * ntiles + t];
  }
  acc = wave_sum_dpp(acc);
  if (lane == 0) {
    const int len = min(block_size, tokens - blk * block_size);
    mass[int64_t(b) * nblk + blk] = acc / (float(heads) * float(tokens)) / float(max(len, 1));
  }
}

template <int D, typename T>
static hipError_t launch_prefill(const PrefillParams& p, int batch, int G, hipStream_t stream) {
  const dim3 grid(unsigned(int64_t(p.nqb) * p.kv_heads * batch));
  if (G == 4)
    hipLaunchKernelGGL((prefill_block_mass_kernel<D, T, 4, true>), grid, dim3(64 * PS_WAVES), 0, stream, p);
  else if (G == PS_MAX_GROUP)
    hipLaunchKernelGGL((prefill_block_mass_kernel<D, T, PS_MAX_GROUP, true>), grid, dim3(64 * PS_WAVES), 0, stream, p);
  else if (G < 4)
    hipLaunchKernelGGL((prefill_block_mass_kernel<D, T, 4, false>), grid, dim3(64 * PS_WAVES), 0, stream, p);
  else
    hipLaunchKernelGGL((prefill_block_mass_kernel<D, T, PS_MAX_GROUP, false>), grid, dim3(64 * PS_WAVES), 0, stream, p);
  return hipGetLastError();
}

}  // namespace tierkv

using namespace tierkv;

extern "C" int64_t tierkv_prefill_block_mass_workspace_bytes(int32_t batch, int32_t num_kv_heads, int32_t tokens) {
  if (batch <= 0 || num_kv_heads <= 0 || tokens <= 0) return -1;
  const int64_t nqb = (tokens + PS_QB - 1) / PS_QB;
  const int64_t ntiles = (tokens + 15) / 16;
  return int64_t(batch) * num_kv_heads * nqb * PS_WAVES * ntiles * 4;
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
  if (batch > 65535) return fail(TIERKV_ERR_UNSUPPORTED, "batch too large");
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
  p.batch = batch;
  if (int64_t(p.nqb) * num_kv_heads * batch > 0x7fffffff) return fail(TIERKV_ERR_UNSUPPORTED, "prefill grid too large");
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
  hipLaunchKernelGGL(prefill_mass_reduce_kernel, dim3(nblk, batch), dim3(64), 0, stream, p.partial,
                     mass, num_kv_heads, p.nqb, p.ntiles, num_heads, tokens, block_size, nblk);
  return check_launch("prefill_mass_reduce_kernel");
}

// WARM-tier codecs on gfx950: demotion (HOT -> WARM quantize + table
// rewrite) and promotion (WARM -> HOT dequantize + table rewrite).
//
// Replaces, batched over blocks, CompactTieredKVTensorPool.demote_to_warm /
// promote_to_hot (tierkv_policy.py:1042-1115), the dense pool's versions
// (329-402), write_warm_block (969-1002) and the codec pair
// quantize_fp16_to_int8 / dequantize_int8_to_fp16 (tierkv_policy.py:21-44).
//
// Bit-exactness: the reference codec is a chain of ATen half ops, each
// computed in fp32 and rounded to fp16; the kernels round after every op
// with __float2half_rn, divide with IEEE __fdiv_rn and round with rintf
// (half to even).  This file is compiled with -ffp-contract=off.

#include "quantize.h"

#include <type_traits>

namespace tierkv {

constexpr int QT = 256;   // threads per quantize workgroup

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float r16(float x) { return __half2float(__float2half_rn(x)); }

__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < QT / 64; ++i) r = fmaxf(r, red[i]);
  __syncthreads();
  return r;
}



// ABSMAX_I8: one workgroup per (job, kv head, K|V) tile.
__global__ __launch_bounds__(QT) void demote_absmax_kernel(QuantJobs q) {
  __shared__ float red[QT / 64];
  const int job = blockIdx.x;
  if (q.n_dev && job >= *q.n_dev) return;
  const int h = blockIdx.y;
  const int kv = blockIdx.z;
  const int64_t si = q.src_index[job];
  const int64_t di = q.dst_slot[job];
  if (si < 0 || si >= q.src_tiles || di < 0 || di >= q.warm_slots) return;
  const int len = min(max(q.lengths[job], 0), q.bs);
  const int64_t E = int64_t(q.bs) * q.D;
  const int64_t valid = int64_t(len) * q.D;
  const __half* src = q.src[kv] + (si * q.kv_heads + h) * E;
  int8_t* dst = reinterpret_cast<int8_t*>(q.warm[kv]) + (di * q.kv_heads + h) * E;

  float amax = 0.f;
  for (int64_t e = threadIdx.x; e < valid; e += QT) amax = fmaxf(amax, fabsf(__half2float(src[e])));
  amax = block_max(amax, red);
  const float s = __fdiv_rn(amax, 127.f);
  for (int64_t e = threadIdx.x; e < E; e += QT) {
    int8_t c = 0;
    if (e < valid && s != 0.f) {
      float r = rintf(__fdiv_rn(__half2float(src[e]), s));
      r = fminf(fmaxf(r, -127.f), 127.f);
      c = static_cast<int8_t>(static_cast<int>(r));
    }
    dst[e] = c;
  }
  if (threadIdx.x == 0) {
    reinterpret_cast<float*>(q.scale[kv])[di * q.kv_heads + h] = s;
    if (q.table_pos && h == 0 && kv == 0) {
      const int32_t pos = q.table_pos[job];
      if (pos >= 0) {
        q.table[pos] = static_cast<int32_t>(di);
        q.states[pos] = WARM;
      }
    }
  }
}

// Vectorised ABSMAX_I8 for head_dim % 8 == 0: each thread owns 8 halves.
__global__ __launch_bounds__(QT) void demote_absmax_vec_kernel(QuantJobs q) {
  __shared__ float red[QT / 64];
  const int job = blockIdx.x;
  if (q.n_dev && job >= *q.n_dev) return;
  const int h = blockIdx.y;
  const int kv = blockIdx.z;
  const int64_t si = q.src_index[job];
  const int64_t di = q.dst_slot[job];
  if (si < 0 || si >= q.src_tiles || di < 0 || di >= q.warm_slots) return;
  const int len = min(max(q.lengths[job], 0), q.bs);
  const int64_t E = int64_t(q.bs) * q.D;
  const int64_t valid = int64_t(len) * q.D;
  const uint4* src = reinterpret_cast<const uint4*>(q.src[kv] + (si * q.kv_heads + h) * E);
  uint2* dst = reinterpret_cast<uint2*>(reinterpret_cast<int8_t*>(q.warm[kv]) + (di * q.kv_heads + h) * E);
  const int64_t nvec = E / 8;

  // Tiles are at most 64 x 256 halves, i.e. <= 8 vectors per thread.
  constexpr int MAXV = 8;
  uint4 x[MAXV];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int64_t vi = threadIdx.x + int64_t(i) * QT;
    if (vi < nvec) {
      x[i] = src[vi];
      if (vi * 8 < valid) {
        const uint32_t w4[4] = {x[i].x, x[i].y, x[i].z, x[i].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          amax = fmaxf(amax, fabsf(half_lo(w4[k])));
          amax = fmaxf(amax, fabsf(half_hi(w4[k])));
        }
      }
    }
  }
  amax = block_max(amax, red);
  const float s = __fdiv_rn(amax, 127.f);
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int64_t vi = threadIdx.x + int64_t(i) * QT;
    if (vi < nvec) {
      uint32_t out[2] = {0u, 0u};
      if (vi * 8 < valid && s != 0.f) {
        const uint32_t w4[4] = {x[i].x, x[i].y, x[i].z, x[i].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          float a = rintf(__fdiv_rn(half_lo(w4[k]), s));
          float b = rintf(__fdiv_rn(half_hi(w4[k]), s));
          a = fminf(fmaxf(a, -127.f), 127.f);
          b = fminf(fmaxf(b, -127.f), 127.f);
          const uint32_t ua = static_cast<uint32_t>(static_cast<int>(a)) & 0xffu;
          const uint32_t ub = static_cast<uint32_t>(static_cast<int>(b)) & 0xffu;
          out[k >> 1] |= (ua | (ub << 8)) << (16 * (k & 1));
        }
      }
      dst[vi] = make_uint2(out[0], out[1]);
    }
  }
  if (threadIdx.x == 0) {
    reinterpret_cast<float*>(q.scale[kv])[di * q.kv_heads + h] = s;
    if (q.table_pos && h == 0 && kv == 0) {
      const int32_t pos = q.table_pos[job];
      if (pos >= 0) {
        q.table[pos] = static_cast<int32_t>(di);
        q.states[pos] = WARM;
      }
    }
  }
}

// Codes of eight elements of an absmax tile (one 16-byte vector, all
// finite): byte k of the result is rintf(x_k / s) clamped to [-127, 127],
// with x_k / s the IEEE (correctly rounded) quotient, computed without the
// division in all but rare cases.  r = RN(1 / s) and q0 = RN(x * r) each
// differ from the exact x / s by a relative 2^-24, so for |x| <= amax
// (|x / s| <= 127 (1 + 2^-24)) |q0 - RN(x / s)| < 2^-16 + 2^-18 < 2^-15.
// rintf changes value only at half-integers; when q0 lies farther than
// 2^-13 from the nearest one, RN(x / s) lies strictly on the same side and
// rintf(q0) == rintf(RN(x / s)), which needs no clamp (|rintf(q0)| <= 127).
// rintf(q0) comes from adding 1.5 * 2^23 (round to nearest even), whose low
// byte is then the two's complement code.  A lane with an element near a
// half-integer (about 2.4e-4 of the elements) recomputes its eight codes
// with the IEEE division.
__device__ __forceinline__ uint2 absmax_codes8(u32x4 w, float s, float r) {
  constexpr float kMagic = 12582912.f;   // 1.5 * 2^23
  float xs[8], t[8], d[8];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    xs[2 * k] = half_lo(w[k]);
    xs[2 * k + 1] = half_hi(w[k]);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float q0 = xs[e] * r;
    t[e] = q0 + kMagic;
    d[e] = q0 - (t[e] - kMagic);   // q0 - rintf(q0), in [-0.5, 0.5]
  }
  const float dmax = fmaxf(fmaxf(fmaxf(fabsf(d[0]), fabsf(d[1])), fmaxf(fabsf(d[2]), fabsf(d[3]))),
                           fmaxf(fmaxf(fabsf(d[4]), fabsf(d[5])), fmaxf(fabsf(d[6]), fabsf(d[7]))));
  if (__builtin_expect(dmax >= 0.5f - 0x1p-13f, 0)) {
#pragma unroll
    for (int e = 0; e < 8; ++e) t[e] = rintf(__fdiv_rn(xs[e], s)) + kMagic;
  }
  uint32_t bt[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) bt[e] = __float_as_uint(t[e]);
  // Low bytes of bt[0..3] -> one word, of bt[4..7] -> the other.
  const uint32_t lo = perm_b32(perm_b32(bt[3], bt[2], 0x0c0c0400u), perm_b32(bt[1], bt[0], 0x0c0c0400u), 0x05040100u);
  const uint32_t hi = perm_b32(perm_b32(bt[7], bt[6], 0x0c0c0400u), perm_b32(bt[5], bt[4], 0x0c0c0400u), 0x05040100u);
  return make_uint2(lo, hi);
}

// The same codes by the IEEE division and the clamp, for tiles holding an
// infinity or a NaN.
__device__ __forceinline__ uint2 absmax_codes8_exact(u32x4 w, float s) {
  uint32_t out[2] = {0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float x = (e & 1) ? half_hi(w[e >> 1]) : half_lo(w[e >> 1]);
    const float n = fminf(fmaxf(rintf(__fdiv_rn(x, s)), -127.f), 127.f);
    out[e >> 2] |= (static_cast<uint32_t>(static_cast<int>(n)) & 0xffu) << (8 * (e & 3));
  }
  return make_uint2(out[0], out[1]);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = max(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), m, 64)));
  return v;
}

typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

// ABSMAX_I8, one wave per (job, K|V, kv head) tile, four tiles (consecutive
// heads of one job) per 256-thread workgroup.  The tile stays in registers
// (NV 16-byte vectors per lane: load i of the wave covers bytes
// [1024 i, 1024 i + 1024) of the tile), the absmax is a wave reduction, and
// each wave stores its codes as 8-byte runs (512 contiguous bytes per store
// instruction).  Needs head_dim % 8 == 0, so every vector lies inside one
// token row, and a tile of at most 64 * NV vectors.
//
// The absmax is taken on the fp16 bit patterns with the sign cleared, which
// order like unsigned integers for finite values, so it is a packed 16-bit
// integer max; a result of 0x7c00 or more flags an infinity or a NaN, and
// such a tile takes the exact path with the fp32 absmax (NaN ignored).
template <int NV>
__global__ __launch_bounds__(QT) void demote_absmax_wave_kernel(QuantJobs q, int32_t n_jobs) {
  const int lane = threadIdx.x & 63;
  const int tiles_per_job = 2 * q.kv_heads;
  const int64_t tile = int64_t(blockIdx.x) * (QT / 64) + (threadIdx.x >> 6);
  const int64_t job = tile / tiles_per_job;
  if (job >= n_jobs) return;
  if (q.n_dev && job >= *q.n_dev) return;
  const int rem = static_cast<int>(tile - job * tiles_per_job);
  const int kv = rem / q.kv_heads;
  const int h = rem - kv * q.kv_heads;
  const int64_t si = q.src_index[job];
  const int64_t di = q.dst_slot[job];
  if (si < 0 || si >= q.src_tiles || di < 0 || di >= q.warm_slots) return;
  const int len = min(max(q.lengths[job], 0), q.bs);
  const int64_t E = int64_t(q.bs) * q.D;
  const int nvec = static_cast<int>(E / 8);
  const int valid_vec = len * q.D / 8;
  const u32x4* src = reinterpret_cast<const u32x4*>(q.src[kv] + (si * q.kv_heads + h) * E);
  u32x2* dst = reinterpret_cast<u32x2*>(reinterpret_cast<int8_t*>(q.warm[kv]) + (di * q.kv_heads + h) * E);

  // Every source byte is read once and every code written once: non-temporal
  // loads and stores.
  u32x4 x[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int vi = i * 64 + lane;
    x[i] = vi < valid_vec ? __builtin_nontemporal_load(src + vi) : u32x4{0u, 0u, 0u, 0u};
  }
  u16x2 m2 = {0, 0};
#pragma unroll
  for (int i = 0; i < NV; ++i) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t a = x[i][k] & 0x7fff7fffu;
      m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2, a));
    }
  }
  const uint32_t abits = wave_max_u32(max(static_cast<uint32_t>(m2[0]), static_cast<uint32_t>(m2[1])));
  if (abits < 0x7c00u) {
    const float amax = __half2float(__ushort_as_half(static_cast<unsigned short>(abits)));
    const float s = __fdiv_rn(amax, 127.f);
    const float r = __fdiv_rn(1.f, s);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int vi = i * 64 + lane;
      if (vi < nvec) {
        const uint2 c = (vi < valid_vec && s != 0.f) ? absmax_codes8(x[i], s, r) : make_uint2(0u, 0u);
        __builtin_nontemporal_store(u32x2{c.x, c.y}, dst + vi);
      }
    }
    if (lane == 0) reinterpret_cast<float*>(q.scale[kv])[di * q.kv_heads + h] = s;
  } else {
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
#pragma unroll
      for (int k = 0; k < 4; ++k) amax = fmaxf(amax, fmaxf(fabsf(half_lo(x[i][k])), fabsf(half_hi(x[i][k]))));
    }
    amax = wave_max(amax);
    const float s = __fdiv_rn(amax, 127.f);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int vi = i * 64 + lane;
      if (vi < nvec) {
        const uint2 c = (vi < valid_vec && s != 0.f) ? absmax_codes8_exact(x[i], s) : make_uint2(0u, 0u);
        dst[vi] = u32x2{c.x, c.y};
      }
    }
    if (lane == 0) reinterpret_cast<float*>(q.scale[kv])[di * q.kv_heads + h] = s;
  }
  if (lane == 0 && q.table_pos && h == 0 && kv == 0) {
    const int32_t pos = q.table_pos[job];
    if (pos >= 0) {
      q.table[pos] = static_cast<int32_t>(di);
      q.states[pos] = WARM;
    }
  }
}

// REF_U8 (quantize_fp16_to_int8, tierkv_policy.py:21-36): one 16-lane group
// per (token, head) row; one workgroup per (job, kv head, K|V) tile.
__global__ __launch_bounds__(QT) void demote_ref_kernel(QuantJobs q) {
  const int job = blockIdx.x;
  if (q.n_dev && job >= *q.n_dev) return;
  const int h = blockIdx.y;
  const int kv = blockIdx.z;
  const int64_t si = q.src_index[job];
  const int64_t di = q.dst_slot[job];
  if (si < 0 || si >= q.src_tiles || di < 0 || di >= q.warm_slots) return;
  const int len = min(max(q.lengths[job], 0), q.bs);
  const int D = q.D;
  const int64_t tile_src = (si * q.kv_heads + h) * int64_t(q.bs);
  const int64_t tile_dst = (di * q.kv_heads + h) * int64_t(q.bs);
  uint8_t* codes = reinterpret_cast<uint8_t*>(q.warm[kv]);
  __half* scale = reinterpret_cast<__half*>(q.scale[kv]);
  __half* zero = reinterpret_cast<__half*>(q.zero[kv]);
  const int sub = threadIdx.x & 15;
  const int rows_per_pass = QT / 16;
  for (int r0 = 0; r0 < q.bs; r0 += rows_per_pass) {
    const int r = r0 + (threadIdx.x >> 4);
    const bool row_ok = r < q.bs;
    const __half* x = q.src[kv] + (tile_src + r) * D;
    float mn = INFINITY, mx = -INFINITY;
    if (row_ok && r < len) {
      for (int d = sub; d < D; d += 16) {
        const float v = __half2float(x[d]);
        mn = fminf(mn, v);
        mx = fmaxf(mx, v);
      }
    }
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) {
      mn = fminf(mn, __shfl_xor(mn, m, 16));
      mx = fmaxf(mx, __shfl_xor(mx, m, 16));
    }
    if (!row_ok) continue;
    uint8_t* out = codes + (tile_dst + r) * D;
    if (r < len) {
      float sc = r16(__fdiv_rn(r16(mx - mn), 255.f));   // (max - min) / 255.0
      if (sc == 0.f) sc = 1.f;                            // torch.where(scale == 0, 1, scale)
      const float zp = r16(-rintf(r16(__fdiv_rn(mn, sc))));   // -round(min / scale)
      for (int d = sub; d < D; d += 16) {
        const float t = rintf(r16(__fdiv_rn(__half2float(x[d]), sc)));   // round(x / scale)
        const float v = fminf(fmaxf(r16(t + zp), 0.f), 255.f);            // + zp, clamp(0, 255)
        out[d] = static_cast<uint8_t>(v);
      }
      if (sub == 0) {
        scale[tile_dst + r] = __float2half_rn(sc);
        zero[tile_dst + r] = __float2half_rn(zp);
      }
    } else if (q.pad_tail) {
      for (int d = sub; d < D; d += 16) out[d] = 0;
      if (sub == 0) {
        scale[tile_dst + r] = __float2half_rn(1.f);
        zero[tile_dst + r] = __float2half_rn(0.f);
      }
    }
  }
  if (threadIdx.x == 0 && q.table_pos && h == 0 && kv == 0) {
    const int32_t pos = q.table_pos[job];
    if (pos >= 0) {
      q.table[pos] = static_cast<int32_t>(di);
      q.states[pos] = WARM;
    }
  }
}


// REF_U8, one wave per (job, K|V, kv head) tile, four tiles per 256-thread
// workgroup.  A token row of D fp16 values is held by R = D / 8 lanes (16
// bytes each, R a power of two), so load i of the wave covers rows
// [64 i / R, 64 (i + 1) / R) of the tile; each row's min and max are reduced
// over its R lanes with xor shuffles, and each lane stores its eight codes as
// one 8-byte run.  The per-element arithmetic is the same op chain as
// demote_ref_kernel.  Needs bs * R <= 64 * NV.
// x / s correctly rounded, given y = RN(1 / s), by Markstein's correction:
// q0 = RN(x y) lies within an ulp of x / s, the residual r = x - q0 s is
// exact by an FMA, and RN(q0 + r y) = RN(x / s); copysign keeps the sign of
// a zero quotient.  tests/native/div_correction_check.c checks it bit for
// bit against the IEEE division for every finite fp16 x and every positive
// finite fp16 s.  x and s must be finite.
__device__ __forceinline__ float div_rn_by(float x, float s, float y) {
  const float q0 = x * y;
  const float r = __builtin_fmaf(-q0, s, x);
  return __builtin_copysignf(__builtin_fmaf(r, y, q0), q0);
}

constexpr float kRcp255 = 1.f / 255.f;   // RN(1 / 255)

// RN(1 / s) for s a positive finite fp16 value held as fp32: the hardware
// reciprocal (within one ulp) and one FMA Newton step.  The residual
// 1 - s y0 is exact, the step leaves y0 (2 - s y0) within 2^-44 of 1 / s,
// and 1 / s lies at least 2^-36 (relative) from every fp32 rounding
// midpoint because s has an 11-bit significand, so the result is the
// correctly rounded reciprocal.  tests/native/rcp_newton_check.c checks
// every such s from both one-ulp neighbours of RN(1 / s) and itself.
__device__ __forceinline__ float rcp_rn_f16_value(float s) {
  const float y0 = __builtin_amdgcn_rcpf(s);
  return __builtin_fmaf(__builtin_fmaf(-s, y0, 1.f), y0, y0);
}

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// Min and max of a token row held by 2^r_log2 consecutive lanes (8 fp16
// values each), returned to every lane of the row.  Packed fp16 min/max
// (minNum semantics, as fminf/fmaxf: a NaN is ignored) over the lane's
// eight values, the max carried negated beside the min so that one packed
// min reduces both; across lanes by DPP row permutes (xor 1 and xor 2 within
// quads, then half-row and row mirrors, each pairing groups that already
// agree), and a shuffle for a 32-lane row.
__device__ __forceinline__ void row_min_max(const u32x4& w, int r_log2, float& mn, float& mx) {
  // The words go through scalars: hipcc (ROCm 7.2) compiles
  // __builtin_bit_cast of a vector element subscript (w[k]) as a read of
  // element 0.
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
  h2 lo = __builtin_bit_cast(h2, ws[0]), hi = lo;
#pragma unroll
  for (int k = 1; k < 4; ++k) {
    const h2 v = __builtin_bit_cast(h2, ws[k]);
    lo = __builtin_elementwise_min(lo, v);
    hi = __builtin_elementwise_max(hi, v);
  }
  h2 m = {__builtin_elementwise_min(lo[0], lo[1]), -__builtin_elementwise_max(hi[0], hi[1])};
  auto step = [&](auto ctrl) {
    const uint32_t o = static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(__builtin_bit_cast(uint32_t, m)), decltype(ctrl)::value, 0xf,
                                    0xf, false));
    m = __builtin_elementwise_min(m, __builtin_bit_cast(h2, o));
  };
  if (r_log2 >= 1) step(std::integral_constant<int, 0xB1>{});    // quad_perm [1, 0, 3, 2]
  if (r_log2 >= 2) step(std::integral_constant<int, 0x4E>{});    // quad_perm [2, 3, 0, 1]
  if (r_log2 >= 3) step(std::integral_constant<int, 0x141>{});   // row_half_mirror
  if (r_log2 >= 4) step(std::integral_constant<int, 0x140>{});   // row_mirror
  if (r_log2 >= 5) {
    const uint32_t o = static_cast<uint32_t>(__shfl_xor(static_cast<int>(__builtin_bit_cast(uint32_t, m)), 16, 64));
    m = __builtin_elementwise_min(m, __builtin_bit_cast(h2, o));
  }
  mn = static_cast<float>(m[0]);
  mx = -static_cast<float>(m[1]);
}

// RL >= 0: r_log2 is RL (the common head dims, so the row reduction has no
// runtime branches); RL < 0: r_log2 comes from the argument.
template <int NV, int RL>
__global__ __launch_bounds__(QT) void demote_ref_wave_kernel(QuantJobs q, int32_t n_jobs, int32_t r_log2_arg) {
  const int r_log2 = RL >= 0 ? RL : r_log2_arg;
  const int lane = threadIdx.x & 63;
  const int tiles_per_job = 2 * q.kv_heads;
  const int64_t tile = int64_t(blockIdx.x) * (QT / 64) + (threadIdx.x >> 6);
  const int64_t job = tile / tiles_per_job;
  if (job >= n_jobs) return;
  if (q.n_dev && job >= *q.n_dev) return;
  const int rem = static_cast<int>(tile - job * tiles_per_job);
  const int kv = rem / q.kv_heads;
  const int h = rem - kv * q.kv_heads;
  const int64_t si = q.src_index[job];
  const int64_t di = q.dst_slot[job];
  if (si < 0 || si >= q.src_tiles || di < 0 || di >= q.warm_slots) return;
  const int len = min(max(q.lengths[job], 0), q.bs);
  const int R = 1 << r_log2;
  const int64_t E = int64_t(q.bs) * q.D;
  const int nvec = q.bs * R;
  const int valid_vec = len * R;
  const u32x4* src = reinterpret_cast<const u32x4*>(q.src[kv] + (si * q.kv_heads + h) * E);
  u32x2* dst = reinterpret_cast<u32x2*>(reinterpret_cast<uint8_t*>(q.warm[kv]) + (di * q.kv_heads + h) * E);
  __half* scale = reinterpret_cast<__half*>(q.scale[kv]) + (di * q.kv_heads + h) * int64_t(q.bs);
  __half* zero = reinterpret_cast<__half*>(q.zero[kv]) + (di * q.kv_heads + h) * int64_t(q.bs);

  u32x4 x[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int vi = i * 64 + lane;
    x[i] = vi < valid_vec ? __builtin_nontemporal_load(src + vi) : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int vi = i * 64 + lane;
    const int row = vi >> r_log2;
    float mn, mx;
    row_min_max(x[i], r_log2, mn, mx);
    if (vi < valid_vec) {
      // The scale is stored, so its quotient is correctly rounded without an
      // IEEE division (div_rn_by); a non-finite operand takes the plain IEEE
      // result.  The other quotients only feed round(): for every finite
      // fp16 x and positive finite fp16 s, rint(RN16(RN32(x * RN32(1 / s))))
      // equals rint(RN16(RN32(x / s))) (tests/native/quotient_rint_check.c
      // checks all 2.0e9 pairs, also with the product rounded to fp16 once:
      // the fp16 quotients differ only below 2^-14, where both round to 0),
      // so one multiply per element by the row's correctly rounded reciprocal
      // gives the reference's integers (y > 0 keeps the sign of a zero).
      const float a = r16(mx - mn);
      float sc = __builtin_isfinite(a) ? div_rn_by(a, 255.f, kRcp255) : a;   // (max - min) / 255.0
      sc = r16(sc);
      if (sc == 0.f) sc = 1.f;                            // torch.where(scale == 0, 1, scale)
      // The words go through scalars (see row_min_max).
      const uint32_t ws[4] = {x[i].x, x[i].y, x[i].z, x[i].w};
      h2 qt[4];
      float qm;
      if (__builtin_isfinite(sc)) {
        const float y = rcp_rn_f16_value(sc);   // sc: a positive finite fp16 value
        qm = mn * y;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const h2 v = __builtin_bit_cast(h2, ws[k]);
          qt[k] = h2{static_cast<_Float16>(static_cast<float>(v[0]) * y),
                     static_cast<_Float16>(static_cast<float>(v[1]) * y)};
        }
      } else {   // a row holding an infinity
        qm = __fdiv_rn(mn, sc);
#pragma unroll
        for (int k = 0; k < 4; ++k)
          qt[k] = h2{static_cast<_Float16>(__fdiv_rn(half_lo(ws[k]), sc)),
                     static_cast<_Float16>(__fdiv_rn(half_hi(ws[k]), sc))};
      }
      const float zp = r16(-rintf(r16(qm)));              // -round(min / scale)
      // round(x / scale) + zp, clamp(0, 255), in fp16 two at a time.  The
      // quotient is rounded to fp16 and then to an integer (rndne on the fp16
      // value equals rintf on it); both terms of the sum are integers of at
      // most 65504 in magnitude, so the fp16 add equals the reference's
      // fp32 add rounded to fp16.  A clamped value v in [0, 255] is the low
      // byte of the fp16 encoding of v + 1024 (exponent 10, unit spacing).
      const _Float16 zh = static_cast<_Float16>(zp);
      uint32_t hb[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        h2 t = __builtin_elementwise_rint(qt[k]);
        t = t + h2{zh, zh};
        t = __builtin_elementwise_min(__builtin_elementwise_max(t, h2{0, 0}), h2{255, 255});
        t = t + h2{1024, 1024};
        hb[k] = __builtin_bit_cast(uint32_t, t);
      }
      // Low bytes of the eight halves: bytes 0 and 2 of each word.
      const uint32_t w[2] = {perm_b32(hb[1], hb[0], 0x06040200u), perm_b32(hb[3], hb[2], 0x06040200u)};
      __builtin_nontemporal_store(u32x2{w[0], w[1]}, dst + vi);
      if ((lane & (R - 1)) == 0) {
        scale[row] = __float2half_rn(sc);
        zero[row] = __float2half_rn(zp);
      }
    } else if (q.pad_tail && vi < nvec) {
      __builtin_nontemporal_store(u32x2{0u, 0u}, dst + vi);
      if ((lane & (R - 1)) == 0) {
        scale[row] = __float2half_rn(1.f);
        zero[row] = __float2half_rn(0.f);
      }
    }
  }
  if (lane == 0 && q.table_pos && h == 0 && kv == 0) {
    const int32_t pos = q.table_pos[job];
    if (pos >= 0) {
      q.table[pos] = static_cast<int32_t>(di);
      q.states[pos] = WARM;
    }
  }
}



// promote_to_hot: dequantize the first `length` tokens of a WARM slot into
// a HOT slot (dequantize_int8_to_fp16, tierkv_policy.py:39-44).
__global__ __launch_bounds__(QT) void promote_kernel(DequantJobs q) {
  const int job = blockIdx.x;
  if (q.n_dev && job >= *q.n_dev) return;
  const int h = blockIdx.y;
  const int kv = blockIdx.z;
  const int64_t si = q.src_slot[job];
  const int64_t di = q.dst_slot[job];
  if (si < 0 || si >= q.warm_slots || di < 0 || di >= q.hot_slots) return;
  const int len = min(max(q.lengths[job], 0), q.bs);
  const int D = q.D;
  const int64_t E = int64_t(len) * D;
  const int64_t src0 = (si * q.kv_heads + h) * int64_t(q.bs);
  const int64_t dst0 = (di * q.kv_heads + h) * int64_t(q.bs);
  __half* out = q.hot[kv] + dst0 * D;
  if (q.warm_format == TIERKV_WARM_ABSMAX_I8) {
    const int8_t* c = reinterpret_cast<const int8_t*>(q.warm[kv]) + src0 * D;
    const float s = reinterpret_cast<const float*>(q.scale[kv])[si * q.kv_heads + h];
    for (int64_t e = threadIdx.x; e < E; e += QT) out[e] = __float2half_rn(float(c[e]) * s);
  } else {
    const uint8_t* c = reinterpret_cast<const uint8_t*>(q.warm[kv]) + src0 * D;
    const __half* sc = reinterpret_cast<const __half*>(q.scale[kv]) + src0;
    const __half* zp = reinterpret_cast<const __half*>(q.zero[kv]) + src0;
    for (int64_t e = threadIdx.x; e < E; e += QT) {
      const int64_t r = e / D;
      const float d = r16(float(c[e]) - __half2float(zp[r]));     // q.to(f16) - zero_point
      out[e] = __float2half_rn(d * __half2float(sc[r]));           // * scale
    }
  }
  if (threadIdx.x == 0 && q.table_pos && h == 0 && kv == 0) {
    const int32_t pos = q.table_pos[job];
    if (pos >= 0) {
      q.table[pos] = static_cast<int32_t>(di);
      q.states[pos] = HOT;
    }
  }
}

// promote_to_hot, one wave per (job, K|V, kv head) tile, four tiles per
// 256-thread workgroup: each lane turns eight codes (one 8-byte load) into
// eight fp16 values (one 16-byte store), with the same per-element
// arithmetic as promote_kernel.  D = 8 R with R a power of two (a vector
// never crosses a token row) and bs * R <= 64 * NV.
template <int NV, int FMT>
__global__ __launch_bounds__(QT) void promote_wave_kernel(DequantJobs q, int32_t n_jobs, int32_t r_log2) {
  const int lane = threadIdx.x & 63;
  const int tiles_per_job = 2 * q.kv_heads;
  const int64_t tile = int64_t(blockIdx.x) * (QT / 64) + (threadIdx.x >> 6);
  const int64_t job = tile / tiles_per_job;
  if (job >= n_jobs) return;
  if (q.n_dev && job >= *q.n_dev) return;
  const int rem = static_cast<int>(tile - job * tiles_per_job);
  const int kv = rem / q.kv_heads;
  const int h = rem - kv * q.kv_heads;
  const int64_t si = q.src_slot[job];
  const int64_t di = q.dst_slot[job];
  if (si < 0 || si >= q.warm_slots || di < 0 || di >= q.hot_slots) return;
  const int len = min(max(q.lengths[job], 0), q.bs);
  const int valid_vec = len << r_log2;
  const int64_t E = int64_t(q.bs) * q.D;
  const int64_t src0 = (si * q.kv_heads + h) * int64_t(q.bs);
  const u32x2* c = reinterpret_cast<const u32x2*>(reinterpret_cast<const uint8_t*>(q.warm[kv]) + src0 * q.D);
  u32x4* out = reinterpret_cast<u32x4*>(q.hot[kv] + (di * q.kv_heads + h) * E);
  // All loads (codes, and the rows' scales and zero points) are issued
  // before any is used.
  u32x2 cw[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int vi = i * 64 + lane;
    cw[i] = vi < valid_vec ? __builtin_nontemporal_load(c + vi) : u32x2{0u, 0u};
  }
  // Reference format: lane t < len loads row t's scale and zero point
  // (bs <= 64); a vector's lanes take them from that lane by a shuffle.
  float sc_row = 0.f, zp_row = 0.f;
  if constexpr (FMT == TIERKV_WARM_REF_U8) {
    if (lane < len) {
      sc_row = __half2float(reinterpret_cast<const __half*>(q.scale[kv])[src0 + lane]);
      zp_row = __half2float(reinterpret_cast<const __half*>(q.zero[kv])[src0 + lane]);
    }
  }
  float s = 0.f;
  if constexpr (FMT == TIERKV_WARM_ABSMAX_I8) s = reinterpret_cast<const float*>(q.scale[kv])[si * q.kv_heads + h];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int vi = i * 64 + lane;
    float sc = 0.f, zp = 0.f;
    if constexpr (FMT == TIERKV_WARM_REF_U8) {
      const int row = min(vi >> r_log2, 63);
      sc = __shfl(sc_row, row, 64);
      zp = __shfl(zp_row, row, 64);
    }
    if (vi >= valid_vec) continue;
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t byte = (cw[i][e >> 2] >> (8 * (e & 3))) & 0xffu;
      float v;
      if constexpr (FMT == TIERKV_WARM_ABSMAX_I8) {
        v = float(static_cast<int8_t>(byte)) * s;
      } else {
        v = r16(float(byte) - zp) * sc;                  // (q.to(f16) - zero_point) * scale
      }
      const uint32_t hb = __half_as_ushort(__float2half_rn(v));
      if (e & 1) o[e >> 1] |= hb << 16;
      else o[e >> 1] = hb;
    }
    __builtin_nontemporal_store(u32x4{o[0], o[1], o[2], o[3]}, out + vi);
  }
  if (lane == 0 && q.table_pos && h == 0 && kv == 0) {
    const int32_t pos = q.table_pos[job];
    if (pos >= 0) {
      q.table[pos] = static_cast<int32_t>(di);
      q.states[pos] = HOT;
    }
  }
}

// log2(head_dim / 8) when head_dim / 8 is a power of two, else -1.
static int row_lanes_log2(int D) {
  if (D % 8 != 0) return -1;
  const int r = D / 8;
  if (r & (r - 1)) return -1;
  int l = 0;
  while ((1 << l) < r) ++l;
  return l;
}

// NV (16-byte vectors per lane) for a tile of nvec vectors, or 0 if above 512.
static int wave_nv(int64_t nvec) {
  return nvec <= 64 ? 1 : nvec <= 128 ? 2 : nvec <= 256 ? 4 : nvec <= 512 ? 8 : 0;
}

int32_t launch_demote(const QuantJobs& q, int n_grid, int32_t warm_format, hipStream_t stream) {
  if (n_grid <= 0) return TIERKV_OK;
  dim3 grid(n_grid, q.kv_heads, 2);
  if (warm_format == TIERKV_WARM_ABSMAX_I8) {
    const bool vec = (q.D % 8 == 0) && aligned16(q.src[0]) && aligned16(q.src[1]) &&
                     (reinterpret_cast<uintptr_t>(q.warm[0]) % 8 == 0) &&
                     (reinterpret_cast<uintptr_t>(q.warm[1]) % 8 == 0);
    const int64_t nvec = int64_t(q.bs) * q.D / 8;
    const int64_t tiles = int64_t(n_grid) * 2 * q.kv_heads;
    const dim3 wgrid(static_cast<unsigned>((tiles + QT / 64 - 1) / (QT / 64)));
    // One wave per tile: the launch's work-item count (64 per tile) must stay below 2^32.
    if (tiles >= (int64_t(1) << 25)) {
      if (vec) hipLaunchKernelGGL(demote_absmax_vec_kernel, grid, dim3(QT), 0, stream, q);
      else hipLaunchKernelGGL(demote_absmax_kernel, grid, dim3(QT), 0, stream, q);
    } else if (vec && nvec <= 64) {
      hipLaunchKernelGGL(demote_absmax_wave_kernel<1>, wgrid, dim3(QT), 0, stream, q, n_grid);
    } else if (vec && nvec <= 128) {
      hipLaunchKernelGGL(demote_absmax_wave_kernel<2>, wgrid, dim3(QT), 0, stream, q, n_grid);
    } else if (vec && nvec <= 256) {
      hipLaunchKernelGGL(demote_absmax_wave_kernel<4>, wgrid, dim3(QT), 0, stream, q, n_grid);
    } else if (vec && nvec <= 512) {
      hipLaunchKernelGGL(demote_absmax_wave_kernel<8>, wgrid, dim3(QT), 0, stream, q, n_grid);
    } else if (vec) hipLaunchKernelGGL(demote_absmax_vec_kernel, grid, dim3(QT), 0, stream, q);
    else hipLaunchKernelGGL(demote_absmax_kernel, grid, dim3(QT), 0, stream, q);
    return check_launch("demote_absmax_kernel");
  }
  if (warm_format == TIERKV_WARM_REF_U8) {
    const int rl = row_lanes_log2(q.D);
    const int64_t tiles = int64_t(n_grid) * 2 * q.kv_heads;
    const int nv = rl < 0 ? 0 : wave_nv(int64_t(q.bs) << rl);
    const bool vec = nv > 0 && q.bs <= 64 && tiles < (int64_t(1) << 25) && aligned16(q.src[0]) && aligned16(q.src[1]) &&
                     reinterpret_cast<uintptr_t>(q.warm[0]) % 8 == 0 && reinterpret_cast<uintptr_t>(q.warm[1]) % 8 == 0;
    if (!vec) {
      hipLaunchKernelGGL(demote_ref_kernel, grid, dim3(QT), 0, stream, q);
      return check_launch("demote_ref_kernel");
    }
    const dim3 wgrid(static_cast<unsigned>((tiles + QT / 64 - 1) / (QT / 64)));
    // Head dim 128 / 64 with 16-token blocks: 16 / 8 lanes per row.
    if (nv == 4 && rl == 4) hipLaunchKernelGGL((demote_ref_wave_kernel<4, 4>), wgrid, dim3(QT), 0, stream, q, n_grid, rl);
    else if (nv == 2 && rl == 3) hipLaunchKernelGGL((demote_ref_wave_kernel<2, 3>), wgrid, dim3(QT), 0, stream, q, n_grid, rl);
    else if (nv == 1) hipLaunchKernelGGL((demote_ref_wave_kernel<1, -1>), wgrid, dim3(QT), 0, stream, q, n_grid, rl);
    else if (nv == 2) hipLaunchKernelGGL((demote_ref_wave_kernel<2, -1>), wgrid, dim3(QT), 0, stream, q, n_grid, rl);
    else if (nv == 4) hipLaunchKernelGGL((demote_ref_wave_kernel<4, -1>), wgrid, dim3(QT), 0, stream, q, n_grid, rl);
    else hipLaunchKernelGGL((demote_ref_wave_kernel<8, -1>), wgrid, dim3(QT), 0, stream, q, n_grid, rl);
    return check_launch("demote_ref_wave_kernel");
  }
  return fail(TIERKV_ERR_INVALID, "unknown warm format");
}

int32_t launch_promote(const DequantJobs& q, int n_grid, hipStream_t stream) {
  if (n_grid <= 0) return TIERKV_OK;
  const int rl = row_lanes_log2(q.D);
  const int64_t tiles = int64_t(n_grid) * 2 * q.kv_heads;
  const int nv = rl < 0 ? 0 : wave_nv(int64_t(q.bs) << rl);
  const bool vec = nv > 0 && q.bs <= 64 && tiles < (int64_t(1) << 25) && aligned16(q.hot[0]) && aligned16(q.hot[1]) &&
                   reinterpret_cast<uintptr_t>(q.warm[0]) % 8 == 0 && reinterpret_cast<uintptr_t>(q.warm[1]) % 8 == 0;
  if (!vec) {
    hipLaunchKernelGGL(promote_kernel, dim3(n_grid, q.kv_heads, 2), dim3(QT), 0, stream, q);
    return check_launch("promote_kernel");
  }
  const dim3 wgrid(static_cast<unsigned>((tiles + QT / 64 - 1) / (QT / 64)));
#define TIERKV_PROMOTE(NV_, FMT_) \
  hipLaunchKernelGGL((promote_wave_kernel<NV_, FMT_>), wgrid, dim3(QT), 0, stream, q, n_grid, rl)
  if (q.warm_format == TIERKV_WARM_ABSMAX_I8) {
    if (nv == 1) TIERKV_PROMOTE(1, TIERKV_WARM_ABSMAX_I8);
    else if (nv == 2) TIERKV_PROMOTE(2, TIERKV_WARM_ABSMAX_I8);
    else if (nv == 4) TIERKV_PROMOTE(4, TIERKV_WARM_ABSMAX_I8);
    else TIERKV_PROMOTE(8, TIERKV_WARM_ABSMAX_I8);
  } else {
    if (nv == 1) TIERKV_PROMOTE(1, TIERKV_WARM_REF_U8);
    else if (nv == 2) TIERKV_PROMOTE(2, TIERKV_WARM_REF_U8);
    else if (nv == 4) TIERKV_PROMOTE(4, TIERKV_WARM_REF_U8);
    else TIERKV_PROMOTE(8, TIERKV_WARM_REF_U8);
  }
#undef TIERKV_PROMOTE
  return check_launch("promote_wave_kernel");
}

}  // namespace tierkv

using namespace tierkv;

extern "C" int32_t tierkv_demote_to_warm(
    const void* src_k, const void* src_v, int64_t src_tiles,
    const int32_t* src_index, const int32_t* dst_slot, const int32_t* lengths, int32_t n,
    void* warm_k, void* warm_v, int64_t warm_slots,
    void* k_scale, void* k_zero, void* v_scale, void* v_zero,
    int32_t warm_format, int32_t pad_tail,
    int32_t* block_table, int32_t* block_states, const int32_t* table_pos,
    int32_t num_kv_heads, int32_t block_size, int32_t head_dim, void* stream_) {
  clear_error();
  if (n < 0) return fail(TIERKV_ERR_INVALID, "negative job count");
  if (n == 0) return TIERKV_OK;
  if (!src_k || !src_v || !src_index || !dst_slot || !lengths || !warm_k || !warm_v || !k_scale || !v_scale)
    return fail(TIERKV_ERR_INVALID, "null pointer");
  if (table_pos && (!block_table || !block_states)) return fail(TIERKV_ERR_INVALID, "table_pos needs block_table and block_states");
  if (num_kv_heads <= 0 || block_size <= 0 || block_size > 64 || head_dim <= 0 || head_dim > 256)
    return fail(TIERKV_ERR_UNSUPPORTED, "block_size must be in [1, 64] and head_dim in [1, 256]");
  if (n > 65535 * 64) return fail(TIERKV_ERR_UNSUPPORTED, "too many demotion jobs in one call");
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  QuantJobs q{};
  q.src[0] = reinterpret_cast<const __half*>(src_k);
  q.src[1] = reinterpret_cast<const __half*>(src_v);
  q.src_tiles = src_tiles;
  q.src_index = src_index;
  q.dst_slot = dst_slot;
  q.lengths = lengths;
  q.warm[0] = warm_k;
  q.warm[1] = warm_v;
  q.warm_slots = warm_slots;
  q.scale[0] = k_scale;
  q.scale[1] = v_scale;
  q.zero[0] = k_zero;
  q.zero[1] = v_zero;
  q.table = block_table;
  q.states = block_states;
  q.table_pos = table_pos;
  q.kv_heads = num_kv_heads;
  q.bs = block_size;
  q.D = head_dim;
  q.pad_tail = pad_tail;
  if (warm_format == TIERKV_WARM_REF_U8 && (!k_zero || !v_zero))
    return fail(TIERKV_ERR_INVALID, "reference format needs zero-point pools");
  return launch_demote(q, n, warm_format, stream);
}

extern "C" int32_t tierkv_promote_to_hot(
    const void* warm_k, const void* warm_v, int64_t warm_slots,
    const void* k_scale, const void* k_zero, const void* v_scale, const void* v_zero,
    const int32_t* src_slot, const int32_t* dst_slot, const int32_t* lengths, int32_t n,
    void* hot_k, void* hot_v, int64_t hot_slots, int32_t warm_format,
    int32_t* block_table, int32_t* block_states, const int32_t* table_pos,
    int32_t num_kv_heads, int32_t block_size, int32_t head_dim, void* stream_) {
  clear_error();
  if (n < 0) return fail(TIERKV_ERR_INVALID, "negative job count");
  if (n == 0) return TIERKV_OK;
  if (!warm_k || !warm_v || !k_scale || !v_scale || !src_slot || !dst_slot || !lengths || !hot_k || !hot_v)
    return fail(TIERKV_ERR_INVALID, "null pointer");
  if (warm_format == TIERKV_WARM_REF_U8 && (!k_zero || !v_zero))
    return fail(TIERKV_ERR_INVALID, "reference format needs zero-point pools");
  if (warm_format != TIERKV_WARM_REF_U8 && warm_format != TIERKV_WARM_ABSMAX_I8)
    return fail(TIERKV_ERR_INVALID, "unknown warm format");
  if (table_pos && (!block_table || !block_states)) return fail(TIERKV_ERR_INVALID, "table_pos needs block_table and block_states");
  if (num_kv_heads <= 0 || block_size <= 0 || block_size > 64 || head_dim <= 0 || head_dim > 256)
    return fail(TIERKV_ERR_UNSUPPORTED, "block_size must be in [1, 64] and head_dim in [1, 256]");
  if (n > 65535 * 64) return fail(TIERKV_ERR_UNSUPPORTED, "too many promotion jobs in one call");
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  DequantJobs q{};
  q.warm[0] = warm_k;
  q.warm[1] = warm_v;
  q.warm_slots = warm_slots;
  q.scale[0] = k_scale;
  q.scale[1] = v_scale;
  q.zero[0] = k_zero;
  q.zero[1] = v_zero;
  q.src_slot = src_slot;
  q.dst_slot = dst_slot;
  q.lengths = lengths;
  q.hot[0] = reinterpret_cast<__half*>(hot_k);
  q.hot[1] = reinterpret_cast<__half*>(hot_v);
  q.hot_slots = hot_slots;
  q.table = block_table;
  q.states = block_states;
  q.table_pos = table_pos;
  q.kv_heads = num_kv_heads;
  q.bs = block_size;
  q.D = head_dim;
  q.warm_format = warm_format;
  return launch_promote(q, n, stream);
}

// Internal helpers shared by the gfx950 kernels and the C ABI shims.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>
#include <string>

#include "../../include/tierkv_hip.h"

namespace tierkv {

constexpr int HOT = 0;
constexpr int WARM = 1;
constexpr int COLD = 2;

// Thread-local message behind tierkv_last_error().
void set_error(const std::string& msg);
void clear_error();

inline int32_t fail(int32_t code, const std::string& msg) {
  set_error(msg);
  return code;
}

inline int32_t check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(TIERKV_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
  }
  return TIERKV_OK;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// A decode call's splits_hint: the split factor, and the deterministic flag.
inline bool hint_deterministic(int32_t hint) { return hint > 0 && (hint & TIERKV_DECODE_DETERMINISTIC) != 0; }
inline int32_t hint_splits(int32_t hint) { return hint > 0 ? (hint & ~TIERKV_DECODE_DETERMINISTIC) : hint; }

// Every argument check of tierkv_decode_attention (decode_attention.hip),
// without a launch: TIERKV_OK or the status that call would return.
int32_t decode_check_args(
    const void* query, int32_t query_dtype, void* out, float* score_sums,
    const int32_t* block_table, const int32_t* block_states, const int32_t* block_lengths,
    int64_t table_stride, int32_t num_blocks,
    const void* hot_k, const void* hot_v, int64_t hot_slots,
    const void* warm_k, const void* warm_v, int64_t warm_slots,
    const void* k_scale, const void* k_zero, const void* v_scale, const void* v_zero,
    int32_t warm_format, int32_t cold_mode,
    int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t block_size, int32_t head_dim,
    int32_t splits_hint, void* workspace, int64_t workspace_bytes);

// ---- device helpers -------------------------------------------------------

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float shfl_xor_f(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}

// The value of lane (lane ^ 16) / (lane ^ 32) through gfx950's lane-swap
// instructions (two VALU operations, no LDS crossbar round trip).
// v_permlane16_swap(a, b) exchanges the odd 16-lane rows of a with the even
// rows of b; with a = b = v, lanes of even rows find their partner's value in
// the second result and lanes of odd rows in the first.  v_permlane32_swap
// does the same with the two 32-lane halves.
__device__ __forceinline__ float xor16_f(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float xor32_f(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor_f(v, m));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += shfl_xor_f(v, m);
  return v;
}

// Inclusive prefix sum over the 64 lanes of a wave (lane i gets the sum of
// lanes 0..i) in DPP moves: four row shifts within each 16-lane row (lanes
// whose source lies outside the row add 0), then the row totals are carried
// by the row broadcasts of lane 15 (into rows 1 and 3) and lane 31 (into
// rows 2 and 3).
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);    // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);    // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);    // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);    // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);   // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);   // row_bcast:31
  return v;
}

// Sum over the 64 lanes of a wave in DPP moves (the same row shifts and
// broadcasts as wave_inclusive_scan, in float), read from lane 63: a fixed
// reduction order with no LDS round trips.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x111, 0xf, 0xf, true));   // row_shr:1
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x112, 0xf, 0xf, true));   // row_shr:2
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x114, 0xf, 0xf, true));   // row_shr:4
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x118, 0xf, 0xf, true));   // row_shr:8
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xa, 0xf, false));  // row_bcast:15
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xc, 0xf, false));  // row_bcast:31
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ f16x4 as_f16x4(uint32_t lo, uint32_t hi);

// v_perm_b32: byte i of the result is byte sel_i of the 8-byte value
// {hi (bytes 4-7), lo (bytes 0-3)}.
__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// Four unsigned bytes u -> four exact fp16 values 1024 + u: each byte is
// placed under the fp16 exponent byte 0x64 (0x6400 | u == 1024 + u).
__device__ __forceinline__ f16x4 u8x4_plus1024(uint32_t w) {
  return as_f16x4(perm_b32(0x64646464u, w, 0x04010400u), perm_b32(0x64646464u, w, 0x04030402u));
}

// Four int8 codes c -> four exact fp16 values 1152 + c (c + 128 == c ^ 0x80).
__device__ __forceinline__ f16x4 i8x4_plus1152(uint32_t w) {
  return u8x4_plus1024(w ^ 0x80808080u);
}

// Byte s of four int8 rows r0..r3 (one code per row) as the four exact fp16
// values 1152 + c: each word takes two rows' bytes under zero high bytes (one
// perm), and one xor with 0x64806480 writes the fp16 exponent byte 0x64 and
// flips the code's top bit (1152 + c == 0x6400 | (c ^ 0x80)).  The same
// values as i8x4_plus1152 of the transposed word, in two instructions per
// word instead of a transpose, an xor and a perm.
__device__ __forceinline__ f16x4 i8_col_plus1152(uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3, int s) {
  const uint32_t sel = 0x0c000c00u | (uint32_t(4 + s) << 16) | uint32_t(s);
  return as_f16x4(perm_b32(r1, r0, sel) ^ 0x64806480u, perm_b32(r3, r2, sel) ^ 0x64806480u);
}

// 4x4 byte transpose: out[s] = {r0.byte s, r1.byte s, r2.byte s, r3.byte s}.
__device__ __forceinline__ void transpose_bytes4x4(uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3,
                                                   uint32_t* out) {
  const uint32_t t01l = perm_b32(r1, r0, 0x05010400u);   // r0.b0 r1.b0 r0.b1 r1.b1
  const uint32_t t01h = perm_b32(r1, r0, 0x07030602u);   // r0.b2 r1.b2 r0.b3 r1.b3
  const uint32_t t23l = perm_b32(r3, r2, 0x05010400u);
  const uint32_t t23h = perm_b32(r3, r2, 0x07030602u);
  out[0] = perm_b32(t23l, t01l, 0x05040100u);
  out[1] = perm_b32(t23l, t01l, 0x07060302u);
  out[2] = perm_b32(t23h, t01h, 0x05040100u);
  out[3] = perm_b32(t23h, t01h, 0x07060302u);
}

__device__ __forceinline__ f16x4 as_f16x4(uint32_t lo, uint32_t hi) {
  union { uint32_t u[2]; f16x4 v; } c;
  c.u[0] = lo;
  c.u[1] = hi;
  return c.v;
}

__device__ __forceinline__ f16x2 as_f16x2(uint32_t w) { return __builtin_bit_cast(f16x2, w); }
__device__ __forceinline__ uint32_t bits_of(f16x2 v) { return __builtin_bit_cast(uint32_t, v); }

__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  __half2 h = __floats2half2_rn(a, b);
  return *reinterpret_cast<uint32_t*>(&h);
}

__device__ __forceinline__ float half_lo(uint32_t w) {
  return __half2float(__ushort_as_half(static_cast<unsigned short>(w & 0xffffu)));
}
__device__ __forceinline__ float half_hi(uint32_t w) {
  return __half2float(__ushort_as_half(static_cast<unsigned short>(w >> 16)));
}

// Sort key of tier-label candidate j with score f: the fp32 bits mapped to
// an unsigned integer of the same order (-0 folded into +0 first, so the two
// compare equal, as floats do) in the high word and ~j in the low word.
// Then K_j > K_i  <=>  s_j > s_i  or  (s_j == s_i and j < i): the order of
// Python's stable descending sort (enforce_budget / enforce_tiered_budget,
// tierkv_policy.py:1391-1477), so a rank is one 64-bit compare per
// candidate.  NaN scores, which have no order as floats, are ordered by
// their bits.
__device__ __forceinline__ uint64_t label_key(float f, int j) {
  const uint32_t b = __float_as_uint(f + 0.0f);
  const uint32_t k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return (static_cast<uint64_t>(k) << 32) | static_cast<uint32_t>(~j);
}

template <typename T> __device__ __forceinline__ float to_f32(T v);
template <> __device__ __forceinline__ float to_f32<__half>(__half v) { return __half2float(v); }
template <> __device__ __forceinline__ float to_f32<__hip_bfloat16>(__hip_bfloat16 v) { return __bfloat162float(v); }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ __half from_f32<__half>(float v) { return __float2half_rn(v); }
template <> __device__ __forceinline__ __hip_bfloat16 from_f32<__hip_bfloat16>(float v) { return __float2bfloat16(v); }

}  // namespace tierkv

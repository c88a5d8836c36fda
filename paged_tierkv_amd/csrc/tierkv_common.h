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

// ---- device helpers -------------------------------------------------------

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float shfl_xor_f(float v, int mask) {
  return __shfl_xor(v, mask, 64);
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

// Four int8 codes packed in a dword -> four exact fp16 values.  The biased
// byte u = c ^ 0x80 = c + 128 is placed under the fp16 exponent of 1024
// (0x6400 | u == 1024 + u exactly), then 1152 is subtracted: exact for every
// code in [-128, 127].
__device__ __forceinline__ void i8x4_to_f16x4(uint32_t w, uint32_t& lo, uint32_t& hi) {
  const uint32_t u = w ^ 0x80808080u;
  lo = (u & 0xffu) | ((u & 0xff00u) << 8) | 0x64006400u;
  hi = ((u >> 16) & 0xffu) | ((u >> 8) & 0xff0000u) | 0x64006400u;
  const __half2 bias = __halves2half2(__float2half(1152.f), __float2half(1152.f));
  __half2 l2 = *reinterpret_cast<__half2*>(&lo);
  __half2 h2 = *reinterpret_cast<__half2*>(&hi);
  l2 = __hsub2(l2, bias);
  h2 = __hsub2(h2, bias);
  lo = *reinterpret_cast<uint32_t*>(&l2);
  hi = *reinterpret_cast<uint32_t*>(&h2);
}

__device__ __forceinline__ f16x4 as_f16x4(uint32_t lo, uint32_t hi) {
  union { uint32_t u[2]; f16x4 v; } c;
  c.u[0] = lo;
  c.u[1] = hi;
  return c.v;
}

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

template <typename T> __device__ __forceinline__ float to_f32(T v);
template <> __device__ __forceinline__ float to_f32<__half>(__half v) { return __half2float(v); }
template <> __device__ __forceinline__ float to_f32<__hip_bfloat16>(__hip_bfloat16 v) { return __bfloat162float(v); }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ __half from_f32<__half>(float v) { return __float2half_rn(v); }
template <> __device__ __forceinline__ __hip_bfloat16 from_f32<__hip_bfloat16>(float v) { return __float2bfloat16(v); }

}  // namespace tierkv

// HBM read ceilings of the box, for the decode kernel's roofline figures:
// a streaming read of a large buffer and a gather of 4 KB tiles in a
// shuffled order (the decode kernel's access pattern: one (block, kv head)
// tile of K or V is 4 KB in fp16), both with the non-temporal load policy
// the decode kernel uses.  A measurement helper for bench.py
// (`--mode ceiling`), built as its own library (libtierkv_ceiling.so); it is
// not part of the tier engine's C ABI.

#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t kNever = 0x9e3779b9u;   // the fold below never equals it for the fill pattern used

__device__ __forceinline__ uint32_t fold(u32x4 v) { return v.x ^ v.y ^ v.z ^ v.w; }

// Grid-stride streaming read, four 16-byte loads in flight per thread.
__global__ __launch_bounds__(512) void stream_read_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                          uint32_t* sink) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4 a = __builtin_nontemporal_load(src + i);
    const u32x4 b = __builtin_nontemporal_load(src + i + stride);
    const u32x4 c = __builtin_nontemporal_load(src + i + 2 * stride);
    const u32x4 d = __builtin_nontemporal_load(src + i + 3 * stride);
    acc ^= fold(a) ^ fold(b) ^ fold(c) ^ fold(d);
  }
  for (; i < n16; i += stride) acc ^= fold(__builtin_nontemporal_load(src + i));
  if (acc == kNever) sink[0] = acc;
}

// Workgroup g reads tiles order[g * per_wg + t], t < per_wg, of 4096 bytes
// each; its eight waves take every eighth tile, two tiles in flight per wave
// (64 lanes x 64 bytes per tile).
__global__ __launch_bounds__(512) void gather_tiles_kernel(const u32x4* __restrict__ src,
                                                           const int32_t* __restrict__ order, int32_t per_wg,
                                                           uint32_t* sink) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int32_t* o = order + int64_t(blockIdx.x) * per_wg;
  uint32_t acc = 0;
  int t = w;
  for (; t + 8 < per_wg; t += 16) {
    const u32x4* p = src + int64_t(o[t]) * 256;
    const u32x4* q = src + int64_t(o[t + 8]) * 256;
    u32x4 a[4], b[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) a[k] = __builtin_nontemporal_load(p + 64 * k + lane);
#pragma unroll
    for (int k = 0; k < 4; ++k) b[k] = __builtin_nontemporal_load(q + 64 * k + lane);
#pragma unroll
    for (int k = 0; k < 4; ++k) acc ^= fold(a[k]) ^ fold(b[k]);
  }
  for (; t < per_wg; t += 8) {
    const u32x4* p = src + int64_t(o[t]) * 256;
#pragma unroll
    for (int k = 0; k < 4; ++k) acc ^= fold(__builtin_nontemporal_load(p + 64 * k + lane));
  }
  if (acc == kNever) sink[0] = acc;
}

}  // namespace

// bytes: a multiple of 16; src 16-byte aligned.  Returns 0 or a hipError_t.
extern "C" __attribute__((visibility("default"))) int32_t tierkv_ceiling_stream_read(
    const void* src, int64_t bytes, uint32_t* sink, int32_t grid, void* stream) {
  if (!src || !sink || bytes <= 0 || bytes % 16 != 0 || grid <= 0) return int32_t(hipErrorInvalidValue);
  hipLaunchKernelGGL(stream_read_kernel, dim3(grid), dim3(512), 0, reinterpret_cast<hipStream_t>(stream),
                     reinterpret_cast<const u32x4*>(src), bytes / 16, sink);
  return int32_t(hipGetLastError());
}

// order: n_wg * per_wg tile indices into src (4096-byte tiles), each below
// src_tiles.  Returns 0 or a hipError_t.
extern "C" __attribute__((visibility("default"))) int32_t tierkv_ceiling_gather(
    const void* src, int64_t src_tiles, const int32_t* order, int32_t n_wg, int32_t per_wg, uint32_t* sink,
    void* stream) {
  if (!src || !order || !sink || src_tiles <= 0 || n_wg <= 0 || per_wg <= 0) return int32_t(hipErrorInvalidValue);
  hipLaunchKernelGGL(gather_tiles_kernel, dim3(n_wg), dim3(512), 0, reinterpret_cast<hipStream_t>(stream),
                     reinterpret_cast<const u32x4*>(src), order, per_wg, sink);
  return int32_t(hipGetLastError());
}

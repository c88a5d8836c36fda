// Job lists of the WARM-tier codec kernels (quantize.hip), shared with the
// runtime kernels that build job lists on the device.
#pragma once

#include "tierkv_common.h"

namespace tierkv {

struct QuantJobs {
  const __half* src[2];      // K, V source tiles [src_tiles, H_kv, bs, D]
  int64_t src_tiles;
  const int32_t* src_index;
  const int32_t* dst_slot;
  const int32_t* lengths;
  void* warm[2];
  int64_t warm_slots;
  void* scale[2];
  void* zero[2];
  int32_t* table;
  int32_t* states;
  const int32_t* table_pos;
  int32_t kv_heads, bs, D, pad_tail;
  const int32_t* n_dev;   // NULL, or the job count in device memory (jobs >= *n_dev exit)
};

struct DequantJobs {
  const void* warm[2];
  int64_t warm_slots;
  const void* scale[2];
  const void* zero[2];
  const int32_t* src_slot;
  const int32_t* dst_slot;
  const int32_t* lengths;
  __half* hot[2];
  int64_t hot_slots;
  int32_t* table;
  int32_t* states;
  const int32_t* table_pos;
  int32_t kv_heads, bs, D, warm_format;
  const int32_t* n_dev;   // NULL, or the job count in device memory (jobs >= *n_dev exit)
};

// Launch demotion jobs [0, n_grid) (format-specific kernel) / promotion jobs;
// with q.n_dev set, jobs at or past *n_dev return at once.
int32_t launch_demote(const QuantJobs& q, int n_grid, int32_t warm_format, hipStream_t stream);
int32_t launch_promote(const DequantJobs& q, int n_grid, hipStream_t stream);

}  // namespace tierkv

"""MI355X-native tiered paged KV-cache decode path (Paged-TierKV drop-in).

Modules:
  tierkv_hip     -- tierkv_decode_attention (drop-in for tierkv_triton)
  tierkv_policy  -- pools, policy engine, runtime, HF cache (drop-in for
                    tierkv_policy)
  block_manager  -- BlockManager over the native C++ implementation
  kernels        -- demotion / promotion / block-score / label kernels
  workloads      -- seeded BASELINE configurations
  build          -- builds libtierkv_hip.so for gfx950
"""

HOT_STATE = 0
WARM_STATE = 1
COLD_STATE = 2

__all__ = ["HOT_STATE", "WARM_STATE", "COLD_STATE"]

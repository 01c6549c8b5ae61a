// Promotion policy -- counterpart of include/cu_roaring/detail/promote.cuh.
#pragma once
#include <hip/hip_runtime_api.h>

#include "cu_roaring/types.hpp"

namespace cu_roaring {

// A threshold N means "a container whose cardinality is > N becomes a bitmap"
// for upload_from_ids' small path; upload() promotes every container when the
// effective threshold is below 4096 (promote.cuh:38-40, src/upload.cpp:104).
static constexpr uint32_t PROMOTE_KEEP_DEFAULT = CR_PROMOTE_KEEP_DEFAULT;
static constexpr uint32_t PROMOTE_ALL = CR_PROMOTE_ALL;
static constexpr uint32_t PROMOTE_AUTO = CR_PROMOTE_AUTO;

// PROMOTE_AUTO -> PROMOTE_ALL when the flat bitset of the universe would take
// more than half of the device's L2 (as reported for one XCD), else
// PROMOTE_KEEP_DEFAULT (promote.cuh:75, src/promote.cu:334-367).
uint32_t resolve_auto_threshold(uint32_t universe_size, int device_id = -1);

// Every array and run container becomes an 8 KiB bitmap; returns a new
// GpuRoaring (promote.cuh:48).  Stream-ordered, no host sync.
GpuRoaring promote_to_bitmap(const GpuRoaring& bm, hipStream_t stream = 0);

// promote_to_bitmap when resolve_auto_threshold gives PROMOTE_ALL and the
// input holds an array or run container, else gpu_roaring_deep_copy
// (promote.cuh:63-64).  Stream-ordered, no host sync.
GpuRoaring promote_auto(const GpuRoaring& bm, hipStream_t stream = 0, int device_id = -1);

// Independent copy, freed with gpu_roaring_free (promote.cuh:83).
GpuRoaring gpu_roaring_deep_copy(const GpuRoaring& bm, hipStream_t stream = 0);

}  // namespace cu_roaring

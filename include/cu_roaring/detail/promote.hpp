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

// PROMOTE_AUTO -> PROMOTE_ALL when the flat bitset of the universe, ceil(U/8)
// bytes, is more than 1/32 of the device's L2 as reported for one XCD (4 MiB on
// MI355X, so U > 2^20), else PROMOTE_KEEP_DEFAULT (promote.cuh:75; the
// reference's rule is 2 ceil(U/8) > L2, src/promote.cu:334-367).  Measured on
// gfx950, the all-bitmap layout answers point queries 1.8-5.4x faster from
// U = 2^20 up, and 10^6 must stay compressed.  Where the container count is
// known, upload() adds the reference's footprint term: under PROMOTE_AUTO it
// keeps the layout when n_containers x 8 KiB x 2 >= ceil(U/8)
// (src/upload.cpp:106-118).  promote_auto() has no such term, as in the
// reference (src/promote.cu:369-385).
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

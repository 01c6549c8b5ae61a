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

}  // namespace cu_roaring

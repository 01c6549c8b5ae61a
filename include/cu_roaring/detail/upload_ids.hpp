// ID and bitset uploads -- counterpart of include/cu_roaring/detail/upload_ids.cuh.
#pragma once
#include <hip/hip_runtime_api.h>

#include "cu_roaring/detail/promote.hpp"
#include "cu_roaring/types.hpp"

namespace cu_roaring {

// Unsorted host ids with duplicates.  More than 1024 ids always produce an
// all-BITMAP result (the threshold only shapes the <= 1024 path), complement
// stored when the distinct count exceeds U/2 (upload_ids.cuh:19-23).
GpuRoaring upload_from_ids(const uint32_t* ids, uint32_t n_ids, uint32_t universe_size, hipStream_t stream = 0,
                           uint32_t bitmap_threshold = PROMOTE_AUTO);

// Same with device-resident ids (no host copy).
GpuRoaring upload_from_device_ids(const uint32_t* d_ids, uint32_t n_ids, uint32_t universe_size,
                                  hipStream_t stream = 0, uint32_t bitmap_threshold = PROMOTE_AUTO);

inline GpuRoaring upload_from_sorted_ids(const uint32_t* ids, uint32_t n_ids, uint32_t universe_size,
                                         hipStream_t stream = 0, uint32_t bitmap_threshold = PROMOTE_AUTO)
{
    return upload_from_ids(ids, n_ids, universe_size, stream, bitmap_threshold);
}

// Flat u32 bitset (bit i = words[i/32] >> (i%32)), n_words = ceil(U/32).
GpuRoaring upload_from_bitset(const uint32_t* host_bitset, uint32_t n_words, uint32_t universe_size,
                              hipStream_t stream = 0);
GpuRoaring upload_from_device_bitset(const uint32_t* d_bitset, uint32_t n_words, uint32_t universe_size,
                                     hipStream_t stream = 0);

}  // namespace cu_roaring

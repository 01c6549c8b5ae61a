// Sorted id export -- counterpart of include/cu_roaring/detail/to_csr.cuh.
#pragma once
#include <hip/hip_runtime_api.h>

#include "cu_roaring/types.hpp"

namespace cu_roaring {

// The stored ids in ascending order as int64 into a buffer of at least
// total_cardinality entries (to_csr.cuh:35); negation is ignored, as in the
// reference.
void enumerate_ids(const GpuRoaring& bitmap, int64_t* output, hipStream_t stream = 0);

// Allocating overload (to_csr.cuh:46): nullptr when total_cardinality is 0;
// the caller frees the buffer with hipFree.
int64_t* enumerate_ids(const GpuRoaring& bitmap, hipStream_t stream = 0);

// The logical cardinality, counted on the device from the containers (no
// reference counterpart): set_operation leaves total_cardinality at 0 and a
// stored card of 0 can mean 65536, so this is the exact count of any result.
// A negated bitmap counts its complement within [0, universe_size).
// Synchronises `stream`.
uint64_t cardinality(const GpuRoaring& bitmap, hipStream_t stream = 0);

}  // namespace cu_roaring

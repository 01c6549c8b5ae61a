// Flat-bitset export -- counterpart of include/cu_roaring/detail/decompress.cuh.
#pragma once
#include <hip/hip_runtime_api.h>

#include "cu_roaring/types.hpp"

namespace cu_roaring {

// ceil(universe_size / 32) words of the flat bitset (complemented within the
// universe when the bitmap is negated); nullptr for an empty universe.  The
// caller frees the buffer with hipFree (decompress.cuh:10-11).
uint32_t* decompress_to_bitset(const GpuRoaring& bitmap, hipStream_t stream = 0);

// Into a pre-allocated buffer of output_size_words words (decompress.cuh:13-16).
void decompress_to_bitset(const GpuRoaring& bitmap, uint32_t* output, uint32_t output_size_words,
                          hipStream_t stream = 0);

}  // namespace cu_roaring

// Roaring portable format (CRoaring's roaring_bitmap_portable_serialize
// layout).  No counterpart in the reference, which reads such files through
// CRoaring and upload() (bench/CMakeLists.txt:89-93).
#pragma once
#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <vector>

#include "cu_roaring/detail/promote.hpp"
#include "cu_roaring/types.hpp"

namespace cu_roaring {

// Bytes portable_serialize writes for `bm`.
size_t portable_size_in_bytes(const GpuRoaring& bm, hipStream_t stream = 0);

// The logical set of `bm` (complemented within [0, U) when negated), each
// container encoded as CRoaring's run_optimize would leave it.  Returns the
// bytes written; throws when `capacity` is too small.
size_t portable_serialize(const GpuRoaring& bm, void* buf, size_t capacity, hipStream_t stream = 0);
std::vector<uint8_t> portable_serialize(const GpuRoaring& bm, hipStream_t stream = 0);

// upload(bm) / upload(bm, U) of a portable-format bitmap held in host memory.
GpuRoaring portable_deserialize(const void* buf, size_t len, hipStream_t stream = 0,
                                uint32_t bitmap_threshold = PROMOTE_AUTO);
GpuRoaring portable_deserialize(const void* buf, size_t len, uint32_t universe_size, hipStream_t stream = 0,
                                uint32_t bitmap_threshold = PROMOTE_AUTO);

}  // namespace cu_roaring

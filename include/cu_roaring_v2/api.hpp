// Batch API -- drop-in for the reference's v2/include/cu_roaring_v2/api.hpp.
//
// CRoaring is not a dependency: upload_batch takes each bitmap's container
// list (cu_roaring::HostContainer, one per high_low_container entry).  With
// CU_ROARING_WITH_CROARING defined and <roaring/roaring.h> available, the
// reference's roaring_bitmap_t* overload is provided on top of it.
#pragma once
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <vector>

#include "cu_roaring_v2/types.hpp"

namespace cu_roaring::v2 {

using HostContainer = cr_host_container;

// N host bitmaps as one device batch: one device block, one host-to-device
// copy, container types kept (api.hpp:22-24).  Synchronises `stream`.
GpuRoaringBatch upload_batch(const HostContainer* const* bitmaps, const uint32_t* n_containers, uint32_t n,
                             hipStream_t stream = 0);

// Releases the device block and the host mirrors; safe on an empty batch.
void free_batch(GpuRoaringBatch& batch);

// Every container becomes an 8 KiB bitmap; a new batch (api.hpp:35-36).
GpuRoaringBatch promote_batch(const GpuRoaringBatch& batch, hipStream_t stream = 0);

// View onto bitmap `bitmap_idx` (api.hpp:42); throws std::out_of_range.
GpuRoaringView make_view(const GpuRoaringBatch& batch, uint32_t bitmap_idx);

// AND of the all-bitmap bitmaps input_indices[0, n_inputs) (a host array)
// into a 1-bitmap batch (api.hpp:52-55).  Throws std::invalid_argument for a
// non-all-bitmap input or n_inputs 0, std::out_of_range for a bad index.
GpuRoaringBatch multi_and(const GpuRoaringBatch& batch, const uint32_t* input_indices, uint32_t n_inputs,
                          hipStream_t stream = 0);

// Bitmap b into device_bitsets[b * words_each, (b + 1) * words_each)
// (api.hpp:62-65); the caller zero-initialises the buffer.
void decompress_batch(const GpuRoaringBatch& batch, uint64_t* device_bitsets, uint64_t words_each,
                      hipStream_t stream = 0);

}  // namespace cu_roaring::v2

#if defined(CU_ROARING_WITH_CROARING)
#include "cu_roaring/detail/upload.hpp"
namespace cu_roaring::v2 {
inline GpuRoaringBatch upload_batch(const roaring_bitmap_t* const* cpus, uint32_t n, hipStream_t stream = 0)
{
    std::vector<std::vector<HostContainer>> lists(n);
    std::vector<const HostContainer*> ptrs(n);
    std::vector<uint32_t> counts(n);
    for (uint32_t b = 0; b < n; ++b) {
        lists[b] = cu_roaring::detail::containers_of(cpus[b]);
        ptrs[b] = lists[b].data();
        counts[b] = static_cast<uint32_t>(lists[b].size());
    }
    return upload_batch(ptrs.data(), counts.data(), n, stream);
}
}  // namespace cu_roaring::v2
#endif

// Device-side membership tests on a batch -- counterpart of
// v2/include/cu_roaring_v2/query.cuh.  Header-only HIP device code, compiled
// into the caller's kernels.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "cu_roaring_v2/types.hpp"

namespace cu_roaring::v2 {

namespace detail {

// Membership of `low` in the container at index `c` of the given metadata
// arrays (query.cuh:15-66): one word for a bitset, a binary search over the
// sorted values of an array, or over the run starts of a run container
// (the last run starting at or below `low`, then its end).
__device__ __forceinline__ bool container_has(const ContainerType* types, const uint32_t* offsets,
                                              const uint16_t* cards, const uint64_t* bitmap_data,
                                              const uint16_t* array_data, const uint16_t* run_data, uint32_t c,
                                              uint32_t low)
{
    const ContainerType t = types[c];
    const uint32_t off = offsets[c];
    if (t == ContainerType::BITMAP) {
        const uint64_t w = bitmap_data[off / 8u + (low >> 6)];
        return (w >> (low & 63u)) & 1ull;
    }
    const uint32_t n = cards[c];
    if (t == ContainerType::ARRAY) {
        const uint16_t* a = array_data + off / 2u;
        uint32_t lo = 0, hi = n;  // first value >= low
        while (lo < hi) {
            const uint32_t mid = (lo + hi) >> 1;
            if (a[mid] < low)
                lo = mid + 1;
            else
                hi = mid;
        }
        return lo < n && a[lo] == low;
    }
    const uint16_t* r = run_data + off / 2u;
    uint32_t lo = 0, hi = n;  // first run whose start > low
    while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (r[2 * mid] <= low)
            lo = mid + 1;
        else
            hi = mid;
    }
    if (lo == 0) return false;
    return low <= static_cast<uint32_t>(r[2 * (lo - 1)]) + r[2 * (lo - 1) + 1];
}

}  // namespace detail

// One bitmap through its view: the key index entry, then the container
// (query.cuh:75-92).
__device__ __forceinline__ bool contains(const GpuRoaringView& v, uint32_t id)
{
    if (v.n_containers == 0) return false;
    const uint32_t high = id >> 16;
    if (high > v.max_key) return false;
    const uint32_t c = v.key_index[high];
    if (c == 0xFFFFu) return false;
    return detail::container_has(v.types, v.offsets, v.cardinalities, v.bitmap_data, v.array_data, v.run_data, c,
                                 id & 0xFFFFu);
}

// Bitmap b of the batch: its CSR slice bounds, the key index entry, then the
// container (query.cuh:97-112).
__device__ __forceinline__ bool contains(const GpuRoaringBatch& batch, uint32_t b, uint32_t id)
{
    if (b >= batch.n_bitmaps) return false;
    const uint32_t k0 = batch.key_index_starts[b];
    const uint32_t k1 = batch.key_index_starts[b + 1];
    const uint32_t high = id >> 16;
    if (high >= k1 - k0) return false;
    const uint32_t local = batch.key_indices[k0 + high];
    if (local == 0xFFFFu) return false;
    return detail::container_has(batch.types, batch.offsets, batch.cardinalities, batch.bitmap_data,
                                 batch.array_data, batch.run_data, batch.container_starts[b] + local, id & 0xFFFFu);
}

}  // namespace cu_roaring::v2

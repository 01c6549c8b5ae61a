// Device-side membership tests on a batch -- the operations of the reference's
// v2/include/cu_roaring_v2/query.cuh (contains on a batch view, and on bitmap
// b of a batch).  Header-only HIP device code, compiled into the caller's
// kernels.
//
// A bitmap of a batch is a slice of CSR metadata over pools the batch shares,
// with a key index of its own.  Seen through the slice's pointers it is an
// ordinary single bitmap, so both operations hand it to the library's own
// cu_roaring::GpuRoaringView, whose contains() resolves the key through the
// key index and tests the container (a bitset word, or a search over an
// array's values or a run container's runs).  A batch stores no complements.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "cu_roaring/device/roaring_view.hpp"
#include "cu_roaring_v2/types.hpp"

namespace cu_roaring::v2 {

namespace detail {

static_assert(static_cast<uint8_t>(ContainerType::ARRAY) == static_cast<uint8_t>(ContainerTypeD::ARRAY) &&
                  static_cast<uint8_t>(ContainerType::BITMAP) == static_cast<uint8_t>(ContainerTypeD::BITMAP) &&
                  static_cast<uint8_t>(ContainerType::RUN) == static_cast<uint8_t>(ContainerTypeD::RUN),
              "the batch and the single-bitmap view share the container type codes");

// The single-bitmap view of a slice: c0 = its first container (global index),
// n its container count, ki its key index (last_key + 1 entries).
__device__ __forceinline__ cu_roaring::GpuRoaringView slice_view(const uint16_t* keys, const ContainerType* types,
                                                                 const uint32_t* offsets, const uint16_t* cards,
                                                                 const uint64_t* bitmap_data,
                                                                 const uint16_t* array_data, const uint16_t* run_data,
                                                                 uint32_t c0, uint32_t n, const uint16_t* ki,
                                                                 uint32_t last_key)
{
    cu_roaring::GpuRoaringView s{};
    s.keys = keys + c0;
    s.types = reinterpret_cast<const cu_roaring::ContainerTypeD*>(types + c0);
    s.offsets = offsets + c0;
    s.cardinalities = cards + c0;
    s.n_containers = n;
    s.bitmap_data = bitmap_data;
    s.array_data = array_data;
    s.run_data = run_data;
    s.key_index = ki;
    s.max_key = last_key;
    s.all_bitmap = false;  // offsets are read, whatever the slice holds
    s.negated = false;
    return s;
}

}  // namespace detail

// One bitmap of a batch through its view (metadata already at its slice).
__device__ __forceinline__ bool contains(const GpuRoaringView& v, uint32_t id)
{
    if (v.n_containers == 0) return false;
    return detail::slice_view(v.keys, v.types, v.offsets, v.cardinalities, v.bitmap_data, v.array_data, v.run_data,
                              0, v.n_containers, v.key_index, v.max_key)
        .contains(id);
}

// Bitmap b of the batch, found by its CSR bounds; an index past the batch or
// a bitmap without keys holds nothing.
__device__ __forceinline__ bool contains(const GpuRoaringBatch& batch, uint32_t b, uint32_t id)
{
    if (b >= batch.n_bitmaps) return false;
    const uint32_t k0 = batch.key_index_starts[b];
    const uint32_t n_keys = batch.key_index_starts[b + 1] - k0;
    if (n_keys == 0) return false;
    const uint32_t c0 = batch.container_starts[b];
    return detail::slice_view(batch.keys, batch.types, batch.offsets, batch.cardinalities, batch.bitmap_data,
                              batch.array_data, batch.run_data, c0, batch.container_starts[b + 1] - c0,
                              batch.key_indices + k0, n_keys - 1)
        .contains(id);
}

}  // namespace cu_roaring::v2

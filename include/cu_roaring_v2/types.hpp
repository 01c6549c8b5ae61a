// Data model of the batch API -- drop-in for the reference's
// v2/include/cu_roaring_v2/types.cuh (same names, field order and types).
#pragma once
#include <cstddef>
#include <cstdint>

#include "cu_roaring_abi.h"

namespace cu_roaring::v2 {

enum class ContainerType : uint8_t { ARRAY = 0, BITMAP = 1, RUN = 2 };

// N Roaring bitmaps in one device block, CSR-style (types.cuh:15-86):
//  - container_starts[b] .. container_starts[b+1] is bitmap b's slice of the
//    concatenated keys / types / offsets / cardinalities (global container ids);
//  - key_indices[key_index_starts[b] + high16] is the LOCAL container index
//    within bitmap b, 0xFFFF when absent (slice length max_key + 1, 0 if empty);
//  - offsets are byte offsets into the pools, which the whole batch shares;
//  - cardinalities: a bitset's count (65536 as 0), an array's count, a run
//    container's number of runs;
//  - host_* mirror per-bitmap scalars in host memory (universe = (max_key+1) << 16).
struct GpuRoaringBatch {
    uint32_t n_bitmaps = 0;
    uint32_t total_containers = 0;
    uint32_t n_bitmap_containers_total = 0;
    uint32_t array_pool_bytes = 0;
    uint32_t run_pool_bytes = 0;

    uint32_t* container_starts = nullptr;
    uint32_t* key_index_starts = nullptr;

    uint16_t* keys = nullptr;
    ContainerType* types = nullptr;
    uint32_t* offsets = nullptr;
    uint16_t* cardinalities = nullptr;

    uint16_t* key_indices = nullptr;

    uint64_t* bitmap_data = nullptr;
    uint16_t* array_data = nullptr;
    uint16_t* run_data = nullptr;

    const uint64_t* host_total_cardinalities = nullptr;
    const uint32_t* host_universe_sizes = nullptr;
    const uint32_t* host_container_starts = nullptr;
    const uint32_t* host_key_index_starts = nullptr;
    const uint32_t* host_n_bitmap_containers = nullptr;

    void* _alloc_base = nullptr;
    void* _host_meta_base = nullptr;
};

// One bitmap of a batch (types.cuh:88-107): metadata pointers already point
// at its slice, so key_index entries index them directly; pools are shared.
struct GpuRoaringView {
    uint32_t n_containers = 0;
    uint32_t max_key = 0;

    uint16_t* keys = nullptr;
    ContainerType* types = nullptr;
    uint32_t* offsets = nullptr;
    uint16_t* cardinalities = nullptr;
    uint16_t* key_index = nullptr;

    uint64_t* bitmap_data = nullptr;
    uint16_t* array_data = nullptr;
    uint16_t* run_data = nullptr;
};

static_assert(sizeof(GpuRoaringBatch) == sizeof(cr_roaring_batch), "GpuRoaringBatch must match the C-ABI struct");
static_assert(offsetof(GpuRoaringBatch, container_starts) == offsetof(cr_roaring_batch, container_starts), "layout");
static_assert(offsetof(GpuRoaringBatch, key_indices) == offsetof(cr_roaring_batch, key_indices), "layout");
static_assert(offsetof(GpuRoaringBatch, host_total_cardinalities) ==
                  offsetof(cr_roaring_batch, host_total_cardinalities),
              "layout");
static_assert(offsetof(GpuRoaringBatch, _host_meta_base) == offsetof(cr_roaring_batch, _host_meta_base), "layout");
static_assert(sizeof(GpuRoaringView) == sizeof(cr_batch_view), "GpuRoaringView must match the C-ABI struct");
static_assert(offsetof(GpuRoaringView, key_index) == offsetof(cr_batch_view, key_index), "layout");
static_assert(offsetof(GpuRoaringView, run_data) == offsetof(cr_batch_view, run_data), "layout");

inline cr_roaring_batch* to_abi(GpuRoaringBatch* b) { return reinterpret_cast<cr_roaring_batch*>(b); }
inline const cr_roaring_batch* to_abi(const GpuRoaringBatch* b) { return reinterpret_cast<const cr_roaring_batch*>(b); }
inline cr_batch_view* to_abi(GpuRoaringView* v) { return reinterpret_cast<cr_batch_view*>(v); }
inline const cr_batch_view* to_abi(const GpuRoaringView* v) { return reinterpret_cast<const cr_batch_view*>(v); }

}  // namespace cu_roaring::v2

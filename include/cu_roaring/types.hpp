// Data model of the MI355X Roaring library -- drop-in for the reference's
// include/cu_roaring/types.cuh:1-65 (same names, same field order and types,
// so a GpuRoaring built by either library has the same bytes).
#pragma once
#include <cstddef>
#include <cstdint>

#include "cu_roaring_abi.h"

namespace cu_roaring {

enum class ContainerType : uint8_t { ARRAY = 0, BITMAP = 1, RUN = 2 };

// GPU-resident Roaring bitmap, structure-of-arrays (types.cuh:15-54).
//  - offsets are BYTE offsets into the per-type pool;
//  - cardinalities are u16: a full container (65536) is stored as 0 and a
//    RUN container stores its number of runs;
//  - key_index[key] = container index or 0xFFFF, length max_key + 1;
//  - negated: the stored set is the complement of the logical set;
//  - _alloc_base: when set, every pointer lives inside this one device block
//    and only it is freed.
struct GpuRoaring {
    uint16_t* keys = nullptr;
    ContainerType* types = nullptr;
    uint32_t* offsets = nullptr;
    uint16_t* cardinalities = nullptr;
    uint32_t n_containers = 0;
    uint32_t universe_size = 0;
    uint64_t total_cardinality = 0;

    uint64_t* bitmap_data = nullptr;
    uint32_t n_bitmap_containers = 0;

    uint16_t* array_data = nullptr;
    uint32_t n_array_containers = 0;
    uint32_t array_pool_bytes = 0;

    uint16_t* run_data = nullptr;
    uint32_t n_run_containers = 0;
    uint32_t run_pool_bytes = 0;

    uint16_t* key_index = nullptr;
    uint32_t max_key = 0;

    bool negated = false;

    void* _alloc_base = nullptr;
};

struct GpuRoaringMeta {  // types.cuh:56-63
    uint32_t n_containers = 0;
    uint32_t n_bitmap_containers = 0;
    uint32_t n_array_containers = 0;
    uint32_t n_run_containers = 0;
    uint32_t universe_size = 0;
    size_t total_bytes = 0;
};

static_assert(sizeof(GpuRoaring) == sizeof(cr_gpu_roaring), "GpuRoaring must match the C-ABI struct");
static_assert(offsetof(GpuRoaring, n_containers) == offsetof(cr_gpu_roaring, n_containers), "layout");
static_assert(offsetof(GpuRoaring, total_cardinality) == offsetof(cr_gpu_roaring, total_cardinality), "layout");
static_assert(offsetof(GpuRoaring, bitmap_data) == offsetof(cr_gpu_roaring, bitmap_data), "layout");
static_assert(offsetof(GpuRoaring, array_pool_bytes) == offsetof(cr_gpu_roaring, array_pool_bytes), "layout");
static_assert(offsetof(GpuRoaring, run_pool_bytes) == offsetof(cr_gpu_roaring, run_pool_bytes), "layout");
static_assert(offsetof(GpuRoaring, key_index) == offsetof(cr_gpu_roaring, key_index), "layout");
static_assert(offsetof(GpuRoaring, negated) == offsetof(cr_gpu_roaring, negated), "layout");
static_assert(offsetof(GpuRoaring, _alloc_base) == offsetof(cr_gpu_roaring, _alloc_base), "layout");
static_assert(sizeof(GpuRoaringMeta) == sizeof(cr_meta), "GpuRoaringMeta must match the C-ABI struct");

inline cr_gpu_roaring* to_abi(GpuRoaring* g) { return reinterpret_cast<cr_gpu_roaring*>(g); }
inline const cr_gpu_roaring* to_abi(const GpuRoaring* g) { return reinterpret_cast<const cr_gpu_roaring*>(g); }

}  // namespace cu_roaring

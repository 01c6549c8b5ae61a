// make_view -- counterpart of include/cu_roaring/device/make_view.cuh:9-27.
// The view aliases the struct's device memory: it must not outlive it.
#pragma once
#include "cu_roaring/device/roaring_view.hpp"
#include "cu_roaring/types.hpp"

namespace cu_roaring {

inline GpuRoaringView make_view(const GpuRoaring& b)
{
    GpuRoaringView v{};
    v.keys = b.keys;
    v.types = reinterpret_cast<const ContainerTypeD*>(b.types);
    v.offsets = b.offsets;
    v.cardinalities = b.cardinalities;
    v.n_containers = b.n_containers;
    v.bitmap_data = b.bitmap_data;
    v.array_data = b.array_data;
    v.run_data = b.run_data;
    v.key_index = b.key_index;
    v.max_key = b.max_key;
    v.all_bitmap = b.n_array_containers == 0 && b.n_run_containers == 0 && b.key_index != nullptr;
    v.negated = b.negated;
    return v;
}

static_assert(sizeof(GpuRoaringView) == sizeof(cr_gpu_roaring_view), "view must match the C-ABI struct");

}  // namespace cu_roaring

// Device query view -- counterpart of include/cu_roaring/device/roaring_view.cuh.
//
// GpuRoaringView is a trivially-copyable POD passed to kernels by value; its
// field order is the reference's (roaring_view.cuh:15-37).  contains() is
// compiled into the caller's kernel (header-only, HIP device code).
#pragma once
#include <cstdint>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define CU_ROARING_DEVICE __device__ __forceinline__
#endif

namespace cu_roaring {

enum class ContainerTypeD : uint8_t { ARRAY = 0, BITMAP = 1, RUN = 2 };

struct GpuRoaringView {
    const uint16_t* keys;
    const ContainerTypeD* types;
    const uint32_t* offsets;
    const uint16_t* cardinalities;
    uint32_t n_containers;

    const uint64_t* bitmap_data;
    const uint16_t* array_data;
    const uint16_t* run_data;

    const uint16_t* key_index;  // key_index[high16] = container idx, 0xFFFF = absent
    uint32_t max_key;

    bool all_bitmap;  // no array/run containers and a key_index: offsets are idx * 8192
    bool negated;     // stored set is the complement; absent keys mean "all ones"

#if defined(__HIPCC__)
    // (id in logical set): stored membership XOR negated.  A key above max_key
    // or absent reports `negated` (roaring_view.cuh:39-75).
    CU_ROARING_DEVICE bool contains(uint32_t id) const
    {
        const uint32_t key = id >> 16;
        const uint32_t low = id & 0xFFFFu;
        if (all_bitmap && key_index) {  // two dependent loads: key_index, then one bitmap word
            if (key > max_key) return negated;
            const uint32_t idx = key_index[key];
            if (idx == 0xFFFFu) return negated;
            const uint64_t w = bitmap_data[(idx << 10) + (low >> 6)];
            return (static_cast<uint32_t>(w >> (low & 63u)) & 1u) ^ static_cast<uint32_t>(negated);
        }
        const int idx = lookup_key(key);
        if (idx < 0) return negated;
        return container_contains(static_cast<uint32_t>(types[idx]), offsets[idx], cardinalities[idx], low) ^
               negated;
    }

    // O(1) direct map when key_index is present, else binary search over keys.
    CU_ROARING_DEVICE int lookup_key(uint32_t key) const
    {
        if (key_index) {
            if (key > max_key) return -1;
            const uint32_t v = key_index[key];
            return v == 0xFFFFu ? -1 : static_cast<int>(v);
        }
        int lo = 0, hi = static_cast<int>(n_containers) - 1;
        while (lo <= hi) {
            const int mid = (lo + hi) >> 1;
            const uint32_t k = keys[mid];
            if (k == key) return mid;
            if (k < key)
                lo = mid + 1;
            else
                hi = mid - 1;
        }
        return -1;
    }

    // Membership of `low` in one container; `byte_offset` indexes the pool of
    // its type, `card` is the element count (array) or run count (run).
    CU_ROARING_DEVICE bool container_contains(uint32_t type, uint32_t byte_offset, uint32_t card,
                                              uint32_t low) const
    {
        if (type == static_cast<uint32_t>(ContainerTypeD::BITMAP)) {
            const uint64_t w = bitmap_data[(byte_offset >> 3) + (low >> 6)];
            return (w >> (low & 63u)) & 1u;
        }
        if (type == static_cast<uint32_t>(ContainerTypeD::ARRAY)) {
            const uint16_t* arr = array_data + (byte_offset >> 1);
            int lo = 0, hi = static_cast<int>(card) - 1;
            while (lo <= hi) {
                const int mid = (lo + hi) >> 1;
                const uint32_t v = arr[mid];
                if (v == low) return true;
                if (v < low)
                    lo = mid + 1;
                else
                    hi = mid - 1;
            }
            return false;
        }
        if (type == static_cast<uint32_t>(ContainerTypeD::RUN)) {  // inclusive [start, start+len]
            const uint16_t* runs = run_data + (byte_offset >> 1);
            int lo = 0, hi = static_cast<int>(card) - 1;
            while (lo <= hi) {
                const int mid = (lo + hi) >> 1;
                const uint32_t s = runs[2 * mid], l = runs[2 * mid + 1];
                if (low < s)
                    hi = mid - 1;
                else if (low > s + l)
                    lo = mid + 1;
                else
                    return true;
            }
            return false;
        }
        return false;
    }
#endif
};

static_assert(sizeof(GpuRoaringView) == 80, "GpuRoaringView layout");

}  // namespace cu_roaring

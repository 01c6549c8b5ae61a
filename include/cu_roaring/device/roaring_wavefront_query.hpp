// Wavefront-cooperative contains for wave64 -- counterpart of
// include/cu_roaring/device/roaring_warp_query.cuh:16-88.
//
// CDNA has no __match_any: lanes sharing a high-16 key are found with ballots
// against a wave-uniform leader key.  Each round takes the lowest pending
// lane's key (readlane), resolves it once with wave-uniform loads, and every
// lane holding that key tests its own low 16 bits.  A wave whose queries all
// share one key (sorted / clustered ids) costs one lookup; when the first
// round matches few lanes the wave falls back to per-lane contains() at once,
// so random ids pay only one extra ballot.
#pragma once
#include "cu_roaring/device/roaring_view.hpp"

#if defined(__HIPCC__)
namespace cu_roaring {

namespace detail {
constexpr int kWaveRounds = 4;     // leader rounds before falling back per lane
constexpr int kMinSharedLanes = 8;  // first-round match count that makes sharing worthwhile
}  // namespace detail

__device__ __forceinline__ bool wavefront_contains(const GpuRoaringView& r, uint32_t id)
{
    const uint32_t key = id >> 16;
    const uint32_t low = id & 0xFFFFu;
    unsigned long long pending = __ballot(1);
    bool done = false;
    bool result = false;
#pragma unroll 1
    for (int round = 0; round < detail::kWaveRounds && pending; ++round) {
        const int leader = __ffsll(static_cast<long long>(pending)) - 1;
        const uint32_t lk = __builtin_amdgcn_readlane(key, leader);  // wave-uniform
        const bool mine = !done && key == lk;
        const unsigned long long members = __ballot(mine);
        if (round == 0 && __popcll(members) < detail::kMinSharedLanes) break;
        // Uniform lookup: every lane computes the same address (one request).
        if (r.all_bitmap && r.key_index) {
            int idx = -1;
            if (lk <= r.max_key) {
                const uint32_t v = r.key_index[lk];
                idx = v == 0xFFFFu ? -1 : static_cast<int>(v);
            }
            if (mine) {
                if (idx < 0) {
                    result = r.negated;
                } else {
                    const uint64_t w = r.bitmap_data[(static_cast<uint32_t>(idx) << 10) + (low >> 6)];
                    result = ((w >> (low & 63u)) & 1u) ^ static_cast<uint32_t>(r.negated);
                }
                done = true;
            }
        } else {
            const int idx = r.lookup_key(lk);
            uint32_t type = 0, off = 0, card = 0;
            if (idx >= 0) {
                type = static_cast<uint32_t>(r.types[idx]);
                off = r.offsets[idx];
                card = r.cardinalities[idx];
            }
            if (mine) {
                result = idx < 0 ? r.negated : (r.container_contains(type, off, card, low) ^ r.negated);
                done = true;
            }
        }
        pending &= ~members;
    }
    if (!done) result = r.contains(id);
    return result;
}

// The reference's name for the cooperative query (roaring_warp_query.cuh:16).
__device__ __forceinline__ bool warp_contains(const GpuRoaringView& r, uint32_t id)
{
    return wavefront_contains(r, id);
}

}  // namespace cu_roaring
#endif

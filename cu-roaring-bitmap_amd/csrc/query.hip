// Batched point queries over the header-only device API.
//
// The reference's benches wrap view.contains() / warp_contains() in one-query-
// per-thread kernels (bench/bench_point_query.cu:123-144).  Here each lane
// keeps QPT independent queries in flight so the dependent key_index -> word
// loads of different queries overlap (random queries are latency-bound gathers
// from the 256 MB Infinity Cache / HBM).  Modes 0 and 1 on an all-bitmap view
// take the view's two-load fast path written without branches; every other
// layout, and modes 2 and 3 on every layout, call GpuRoaringView::contains and
// wavefront_contains unchanged.
#include <algorithm>
#include <cstring>

#include "cu_roaring/device/roaring_view.hpp"
#include "cu_roaring/device/roaring_wavefront_query.hpp"
#include "internal.hpp"

namespace crimpl {

using cu_roaring::GpuRoaringView;

constexpr int Q_NT = 256;
constexpr int QPT = 8;

// The id stream and the answers use nontemporal loads and stores, so they do
// not evict the containers (reused by every query) from the caches.
// WAVE: when every lane of the wave queries the same key, the key_index entry
// is read once with a wave-uniform (scalar) load -- wavefront_contains'
// amortisation -- while the QPT queries of a lane stay independent.
template <bool WAVE>
__global__ __launch_bounds__(Q_NT) void contains_allbitmap(GpuRoaringView v, const uint32_t* __restrict__ ids,
                                                           uint64_t n, uint32_t* __restrict__ out)
{
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * Q_NT * QPT;
    const uint32_t neg = v.negated ? 1u : 0u;
    for (uint64_t blk = static_cast<uint64_t>(blockIdx.x) * Q_NT * QPT; blk < n; blk += stride) {
        uint32_t id[QPT], idx[QPT];
#pragma unroll
        for (int q = 0; q < QPT; ++q) {
            const uint64_t i = blk + static_cast<uint64_t>(q) * Q_NT + threadIdx.x;
            id[q] = i < n ? __builtin_nontemporal_load(ids + i) : 0u;
        }
#pragma unroll
        for (int q = 0; q < QPT; ++q) {
            const uint32_t key = id[q] >> 16;
            if (WAVE) {
                const uint32_t k0 = __builtin_amdgcn_readfirstlane(key);
                if (__ballot(key != k0) == 0ull) {  // wave-uniform key
                    const uint32_t x = v.key_index[min(k0, v.max_key)];
                    idx[q] = k0 > v.max_key ? 0xFFFFu : x;
                    continue;
                }
            }
            const uint32_t k = min(key, v.max_key);
            const uint32_t x = v.key_index[k];
            idx[q] = key > v.max_key ? 0xFFFFu : x;
        }
#pragma unroll
        for (int q = 0; q < QPT; ++q) {
            const uint64_t i = blk + static_cast<uint64_t>(q) * Q_NT + threadIdx.x;
            uint32_t r = neg;
            if (idx[q] != 0xFFFFu) {
                const uint32_t low = id[q] & 0xFFFFu;
                const uint64_t w = v.bitmap_data[(idx[q] << 10) + (low >> 6)];
                r = (static_cast<uint32_t>(w >> (low & 63u)) & 1u) ^ neg;
            }
            if (i < n) __builtin_nontemporal_store(r, out + i);
        }
    }
}

template <int MODE>
__global__ __launch_bounds__(Q_NT) void contains_general(GpuRoaringView v, const uint32_t* __restrict__ ids,
                                                         uint64_t n, uint32_t* __restrict__ out)
{
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * Q_NT * QPT;
    for (uint64_t blk = static_cast<uint64_t>(blockIdx.x) * Q_NT * QPT; blk < n; blk += stride) {
#pragma unroll
        for (int q = 0; q < QPT; ++q) {
            const uint64_t i = blk + static_cast<uint64_t>(q) * Q_NT + threadIdx.x;
            if (i < n) {
                const uint32_t id = __builtin_nontemporal_load(ids + i);
                const bool r = MODE == CR_QUERY_WAVEFRONT ? cu_roaring::wavefront_contains(v, id) : v.contains(id);
                __builtin_nontemporal_store(r ? 1u : 0u, out + i);
            }
        }
    }
}

}  // namespace crimpl

using namespace crimpl;

extern "C" int cr_contains_batch(const cr_gpu_roaring_view* view, const uint32_t* d_ids, uint64_t n, uint32_t* d_out,
                                 uint32_t mode, cr_stream_t stream)
{
    if (!view || (n && (!d_ids || !d_out)) || mode > CR_QUERY_CONTAINS_API) {
        set_error("cr_contains_batch: invalid argument");
        return CR_ERR_INVALID;
    }
    if (n == 0) return CR_OK;
    GpuRoaringView v;
    static_assert(sizeof(v) == sizeof(*view), "view layout");
    std::memcpy(&v, view, sizeof(v));
    hipStream_t s = as_stream(stream);
    const uint32_t cus = num_cus();
    const uint64_t per_block = static_cast<uint64_t>(Q_NT) * QPT;
    const unsigned grid = static_cast<unsigned>(
        std::max<uint64_t>(1, std::min<uint64_t>((n + per_block - 1) / per_block, static_cast<uint64_t>(cus) * 16u)));
    {
        CR_TIMED("contains", s);
        if (v.all_bitmap && mode == CR_QUERY_CONTAINS) {
            contains_allbitmap<false><<<grid, Q_NT, 0, s>>>(v, d_ids, n, d_out);
        } else if (v.all_bitmap && mode == CR_QUERY_WAVEFRONT) {
            contains_allbitmap<true><<<grid, Q_NT, 0, s>>>(v, d_ids, n, d_out);
        } else if (mode == CR_QUERY_WAVEFRONT || mode == CR_QUERY_WAVEFRONT_API) {
            contains_general<CR_QUERY_WAVEFRONT><<<grid, Q_NT, 0, s>>>(v, d_ids, n, d_out);
        } else {
            contains_general<CR_QUERY_CONTAINS><<<grid, Q_NT, 0, s>>>(v, d_ids, n, d_out);
        }
    }
    CR_LAUNCH_CHECK();
    return CR_OK;
}

// Host-Roaring upload -- counterpart of include/cu_roaring/detail/upload.cuh.
//
// CRoaring is not a dependency of this library.  The upload() overloads take
// the container list a roaring_bitmap_t holds (HostContainer, one per
// high_low_container entry); when CU_ROARING_WITH_CROARING is defined and
// <roaring/roaring.h> is available, the reference's roaring_bitmap_t*
// overloads are provided on top of them (see the adapter below).
#pragma once
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <vector>

#include "cu_roaring/detail/promote.hpp"
#include "cu_roaring/types.hpp"

namespace cu_roaring {

using HostContainer = cr_host_container;  // key, CRoaring typecode (1/2/3), cardinality|n_runs, data

// upload(cpu_bitmap, stream, thr) -- universe inferred from the last key, no complement.
GpuRoaring upload(const HostContainer* containers, uint32_t n, hipStream_t stream = 0,
                  uint32_t bitmap_threshold = PROMOTE_AUTO);
// upload(cpu_bitmap, U, stream, thr) -- stores the complement (negated=true)
// when the cardinality exceeds U/2.
GpuRoaring upload(const HostContainer* containers, uint32_t n, uint32_t universe_size, hipStream_t stream = 0,
                  uint32_t bitmap_threshold = PROMOTE_AUTO);

void gpu_roaring_free(GpuRoaring& bitmap);
void gpu_roaring_free_async(GpuRoaring& bitmap, hipStream_t stream);

GpuRoaringMeta get_meta(const HostContainer* containers, uint32_t n);

// Complement of a host container list over [0, universe_size): what
// roaring_bitmap_flip_inplace produces, retyped array (<= 4096) / bitset.
// `storage` owns the payloads of the returned containers.
std::vector<HostContainer> complement_containers(const HostContainer* containers, uint32_t n,
                                                 uint32_t universe_size, std::vector<std::vector<uint64_t>>& storage);

}  // namespace cu_roaring

#if defined(CU_ROARING_WITH_CROARING)
// The container structs live in CRoaring's internal headers, as in
// src/upload.cpp:5-18 (roaring::internal in CRoaring v4.x).
#include <roaring/roaring.h>
#include <roaring/containers/array.h>
#include <roaring/containers/bitset.h>
#include <roaring/containers/run.h>
namespace cu_roaring {
namespace detail {
// Walk roaring_bitmap_t::high_low_container (src/upload.cpp:31-71).
inline std::vector<HostContainer> containers_of(const roaring_bitmap_t* bm)
{
    const roaring_array_t& ra = bm->high_low_container;
    std::vector<HostContainer> out(static_cast<size_t>(ra.size));
    for (int32_t i = 0; i < ra.size; ++i) {
        out[i].key = ra.keys[i];
        out[i].typecode = ra.typecodes[i];
        const void* c = ra.containers[i];
        if (ra.typecodes[i] == CR_TC_BITSET) {
            auto* b = static_cast<const roaring::internal::bitset_container_t*>(c);
            out[i].cardinality = b->cardinality;
            out[i].data = b->words;
        } else if (ra.typecodes[i] == CR_TC_ARRAY) {
            auto* a = static_cast<const roaring::internal::array_container_t*>(c);
            out[i].cardinality = a->cardinality;
            out[i].data = a->array;
        } else {
            auto* r = static_cast<const roaring::internal::run_container_t*>(c);
            out[i].cardinality = r->n_runs;
            out[i].data = r->runs;
        }
    }
    return out;
}
}  // namespace detail

inline GpuRoaring upload(const roaring_bitmap_t* bm, hipStream_t stream = 0, uint32_t thr = PROMOTE_AUTO)
{
    auto c = detail::containers_of(bm);
    return upload(c.data(), static_cast<uint32_t>(c.size()), stream, thr);
}

inline GpuRoaring upload(const roaring_bitmap_t* bm, uint32_t universe_size, hipStream_t stream = 0,
                         uint32_t thr = PROMOTE_AUTO)
{
    uint64_t card = roaring_bitmap_get_cardinality(bm);
    if (card > static_cast<uint64_t>(universe_size) / 2) {  // src/upload.cpp:300-313
        roaring_bitmap_t* comp = roaring_bitmap_copy(bm);
        roaring_bitmap_flip_inplace(comp, 0, static_cast<uint64_t>(universe_size));
        auto c = detail::containers_of(comp);
        GpuRoaring out;
        int rc = cr_upload_containers(c.data(), static_cast<uint32_t>(c.size()), universe_size, true, card,
                                      stream, thr, to_abi(&out));
        roaring_bitmap_free(comp);
        throw_on_error(rc, "upload");
        return out;
    }
    auto c = detail::containers_of(bm);
    GpuRoaring out;
    throw_on_error(cr_upload_containers(c.data(), static_cast<uint32_t>(c.size()), universe_size, false, card,
                                        stream, thr, to_abi(&out)),
                   "upload");
    return out;
}

inline GpuRoaringMeta get_meta(const roaring_bitmap_t* bm)
{
    auto c = detail::containers_of(bm);
    return get_meta(c.data(), static_cast<uint32_t>(c.size()));
}
}  // namespace cu_roaring
#endif

// Host C++ API (namespace cu_roaring) over the C-ABI -- the drop-in surface of
// the reference's include/cu_roaring/detail/*.cuh.  Each call forwards to the
// matching cr_* entry point and throws std::runtime_error on failure (the
// reference's CUDA_CHECK contract, include/cu_roaring/detail/utils.cuh:9-18).
#include <algorithm>
#include <cstring>
#include <vector>

#include "cu_roaring/cu_roaring.hpp"

namespace cu_roaring {

static cr_stream_t S(hipStream_t s) { return reinterpret_cast<cr_stream_t>(s); }

uint32_t resolve_auto_threshold(uint32_t universe_size, int device_id)
{
    uint32_t t = 0;
    throw_on_error(cr_resolve_auto_threshold(universe_size, device_id, &t), "resolve_auto_threshold");
    return t;
}

GpuRoaring promote_to_bitmap(const GpuRoaring& bm, hipStream_t stream)
{
    GpuRoaring r;
    throw_on_error(cr_promote_to_bitmap(to_abi(&bm), S(stream), to_abi(&r)), "promote_to_bitmap");
    return r;
}

GpuRoaring promote_auto(const GpuRoaring& bm, hipStream_t stream, int device_id)
{
    GpuRoaring r;
    throw_on_error(cr_promote_auto(to_abi(&bm), S(stream), device_id, to_abi(&r)), "promote_auto");
    return r;
}

GpuRoaring gpu_roaring_deep_copy(const GpuRoaring& bm, hipStream_t stream)
{
    GpuRoaring r;
    throw_on_error(cr_deep_copy(to_abi(&bm), S(stream), to_abi(&r)), "gpu_roaring_deep_copy");
    return r;
}

uint32_t* decompress_to_bitset(const GpuRoaring& bitmap, hipStream_t stream)
{
    uint32_t* out = nullptr;
    uint32_t n_words = 0;
    throw_on_error(cr_decompress_to_bitset_alloc(to_abi(&bitmap), S(stream), &out, &n_words), "decompress_to_bitset");
    return out;
}

void decompress_to_bitset(const GpuRoaring& bitmap, uint32_t* output, uint32_t output_size_words, hipStream_t stream)
{
    throw_on_error(cr_decompress_to_bitset(to_abi(&bitmap), output, output_size_words, S(stream)),
                   "decompress_to_bitset");
}

void enumerate_ids(const GpuRoaring& bitmap, int64_t* output, hipStream_t stream)
{
    throw_on_error(cr_enumerate_ids(to_abi(&bitmap), output, UINT64_MAX, S(stream)), "enumerate_ids");
}

int64_t* enumerate_ids(const GpuRoaring& bitmap, hipStream_t stream)
{
    int64_t* out = nullptr;
    throw_on_error(cr_enumerate_ids_alloc(to_abi(&bitmap), S(stream), &out, nullptr), "enumerate_ids");
    return out;
}

GpuRoaring upload_from_ids(const uint32_t* ids, uint32_t n_ids, uint32_t universe_size, hipStream_t stream,
                           uint32_t bitmap_threshold)
{
    GpuRoaring r;
    throw_on_error(cr_upload_from_ids(ids, n_ids, universe_size, S(stream), bitmap_threshold, to_abi(&r)),
                   "upload_from_ids");
    return r;
}

GpuRoaring upload_from_device_ids(const uint32_t* d_ids, uint32_t n_ids, uint32_t universe_size, hipStream_t stream,
                                  uint32_t bitmap_threshold)
{
    GpuRoaring r;
    throw_on_error(cr_upload_from_device_ids(d_ids, n_ids, universe_size, S(stream), bitmap_threshold, to_abi(&r)),
                   "upload_from_device_ids");
    return r;
}

GpuRoaring upload_from_bitset(const uint32_t* host_bitset, uint32_t n_words, uint32_t universe_size,
                              hipStream_t stream)
{
    GpuRoaring r;
    throw_on_error(cr_upload_from_bitset(host_bitset, n_words, universe_size, S(stream), to_abi(&r)),
                   "upload_from_bitset");
    return r;
}

GpuRoaring upload_from_device_bitset(const uint32_t* d_bitset, uint32_t n_words, uint32_t universe_size,
                                     hipStream_t stream)
{
    GpuRoaring r;
    throw_on_error(cr_upload_from_device_bitset(d_bitset, n_words, universe_size, S(stream), to_abi(&r)),
                   "upload_from_device_bitset");
    return r;
}

static uint64_t host_cardinality(const HostContainer* c, uint32_t n)
{
    uint64_t t = 0;
    for (uint32_t i = 0; i < n; ++i) {
        if (c[i].typecode != CR_TC_RUN) {
            t += static_cast<uint64_t>(c[i].cardinality);
        } else {
            const uint16_t* r = static_cast<const uint16_t*>(c[i].data);
            for (int32_t k = 0; k < c[i].cardinality; ++k) t += static_cast<uint64_t>(r[2 * k + 1]) + 1u;
        }
    }
    return t;
}

GpuRoaring upload(const HostContainer* containers, uint32_t n, hipStream_t stream, uint32_t bitmap_threshold)
{
    GpuRoaring r;
    throw_on_error(cr_upload_containers(containers, n, 0, false, 0, S(stream), bitmap_threshold, to_abi(&r)),
                   "upload");
    return r;
}

std::vector<HostContainer> complement_containers(const HostContainer* c, uint32_t n, uint32_t universe,
                                                 std::vector<std::vector<uint64_t>>& storage)
{
    // roaring_bitmap_flip_inplace(bm, 0, U): every key of [0, ceil(U/65536))
    // is inverted inside [0, U); the result is retyped array (<= 4096) or bitset.
    std::vector<HostContainer> out;
    storage.clear();
    if (universe == 0) return out;
    const uint32_t last_key = (universe - 1u) >> 16;
    uint32_t j = 0;
    std::vector<uint64_t> bits(1024);
    for (uint32_t key = 0; key <= last_key; ++key) {
        std::fill(bits.begin(), bits.end(), 0ull);
        while (j < n && c[j].key < key) ++j;
        if (j < n && c[j].key == key) {
            const HostContainer& h = c[j];
            if (h.typecode == CR_TC_BITSET) {
                std::memcpy(bits.data(), h.data, 8192);
            } else if (h.typecode == CR_TC_ARRAY) {
                const uint16_t* a = static_cast<const uint16_t*>(h.data);
                for (int32_t i = 0; i < h.cardinality; ++i) bits[a[i] >> 6] |= 1ull << (a[i] & 63u);
            } else {
                const uint16_t* r = static_cast<const uint16_t*>(h.data);
                for (int32_t k = 0; k < h.cardinality; ++k) {
                    const uint32_t s = r[2 * k], e = std::min<uint32_t>(0xFFFFu, s + r[2 * k + 1]);
                    for (uint32_t v = s; v <= e; ++v) bits[v >> 6] |= 1ull << (v & 63u);
                }
            }
        }
        const uint64_t valid = std::min<uint64_t>(65536u, static_cast<uint64_t>(universe) - (uint64_t(key) << 16));
        uint32_t card = 0;
        for (uint32_t w = 0; w < 1024u; ++w) {
            uint64_t m = ~0ull;
            const uint64_t lo = uint64_t(w) * 64u;
            if (lo >= valid)
                m = 0;
            else if (lo + 64u > valid)
                m = (1ull << (valid - lo)) - 1ull;
            bits[w] = ~bits[w] & m;
            card += static_cast<uint32_t>(__builtin_popcountll(bits[w]));
        }
        if (card == 0) continue;
        HostContainer hc{};
        hc.key = static_cast<uint16_t>(key);
        hc.cardinality = static_cast<int32_t>(card);
        if (card <= 4096u) {
            std::vector<uint64_t> store((card + 3) / 4);
            uint16_t* a = reinterpret_cast<uint16_t*>(store.data());
            uint32_t k = 0;
            for (uint32_t w = 0; w < 1024u; ++w)
                for (uint64_t x = bits[w]; x; x &= x - 1) a[k++] = static_cast<uint16_t>(w * 64u + __builtin_ctzll(x));
            hc.typecode = CR_TC_ARRAY;
            storage.push_back(std::move(store));
        } else {
            hc.typecode = CR_TC_BITSET;
            storage.push_back(bits);
        }
        out.push_back(hc);
    }
    for (size_t i = 0; i < out.size(); ++i) out[i].data = storage[i].data();
    return out;
}

GpuRoaring upload(const HostContainer* containers, uint32_t n, uint32_t universe_size, hipStream_t stream,
                  uint32_t bitmap_threshold)
{
    const uint64_t card = host_cardinality(containers, n);
    GpuRoaring r;
    if (card > static_cast<uint64_t>(universe_size) / 2u) {  // src/upload.cpp:300-313
        std::vector<std::vector<uint64_t>> storage;
        auto comp = complement_containers(containers, n, universe_size, storage);
        throw_on_error(cr_upload_containers(comp.data(), static_cast<uint32_t>(comp.size()), universe_size, true, card,
                                            S(stream), bitmap_threshold, to_abi(&r)),
                       "upload");
        return r;
    }
    throw_on_error(
        cr_upload_containers(containers, n, universe_size, false, card, S(stream), bitmap_threshold, to_abi(&r)),
        "upload");
    return r;
}

void gpu_roaring_free(GpuRoaring& bitmap) { throw_on_error(cr_free(to_abi(&bitmap)), "gpu_roaring_free"); }

void gpu_roaring_free_async(GpuRoaring& bitmap, hipStream_t stream)
{
    throw_on_error(cr_free_async(to_abi(&bitmap), S(stream)), "gpu_roaring_free_async");
}

GpuRoaringMeta get_meta(const HostContainer* containers, uint32_t n)
{
    GpuRoaringMeta m;
    throw_on_error(cr_get_meta(containers, n, reinterpret_cast<cr_meta*>(&m)), "get_meta");
    return m;
}

GpuRoaring set_operation(const GpuRoaring& a, const GpuRoaring& b, SetOp op, hipStream_t stream)
{
    GpuRoaring r;
    throw_on_error(cr_set_operation(to_abi(&a), to_abi(&b), static_cast<uint32_t>(op), S(stream), to_abi(&r)),
                   "set_operation");
    return r;
}

GpuRoaring multi_and(const GpuRoaring* bitmaps, uint32_t count, hipStream_t stream)
{
    GpuRoaring r;
    throw_on_error(cr_multi_and(reinterpret_cast<const cr_gpu_roaring*>(bitmaps), count, S(stream), to_abi(&r)),
                   "multi_and");
    return r;
}

void topk_filtered(const float* d_base, uint64_t n_base, const float* d_queries, uint32_t n_q, uint32_t dim,
                   const GpuRoaring* filter, uint32_t k, float* d_out_dist, int64_t* d_out_ids, hipStream_t stream)
{
    throw_on_error(cr_topk_filtered(d_base, n_base, d_queries, n_q, dim, filter ? to_abi(filter) : nullptr, k,
                                    d_out_dist, d_out_ids, S(stream)),
                   "topk_filtered");
}

}  // namespace cu_roaring

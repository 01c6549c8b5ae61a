// Host C++ API (namespace cu_roaring) over the C-ABI -- the drop-in surface of
// the reference's include/cu_roaring/detail/*.cuh.  Each call forwards to the
// matching cr_* entry point and throws std::runtime_error on failure (the
// reference's CUDA_CHECK contract, include/cu_roaring/detail/utils.cuh:9-18).
#include <algorithm>
#include <cstring>
#include <vector>

#include "cu_roaring/cu_roaring.hpp"

namespace crimpl {
void set_error(const char* fmt, ...);  // the C ABI's thread-local error message (csrc/runtime.hip)
}

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

uint64_t cardinality(const GpuRoaring& bitmap, hipStream_t stream)
{
    uint64_t n = 0;
    throw_on_error(cr_cardinality(to_abi(&bitmap), S(stream), &n), "cardinality");
    return n;
}

size_t portable_size_in_bytes(const GpuRoaring& bm, hipStream_t stream)
{
    size_t n = 0;
    throw_on_error(cr_portable_size_in_bytes(to_abi(&bm), S(stream), &n), "portable_size_in_bytes");
    return n;
}

size_t portable_serialize(const GpuRoaring& bm, void* buf, size_t capacity, hipStream_t stream)
{
    size_t w = 0;
    throw_on_error(cr_portable_serialize(to_abi(&bm), S(stream), buf, capacity, &w), "portable_serialize");
    return w;
}

std::vector<uint8_t> portable_serialize(const GpuRoaring& bm, hipStream_t stream)
{
    std::vector<uint8_t> out(portable_size_in_bytes(bm, stream));
    out.resize(portable_serialize(bm, out.data(), out.size(), stream));
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

// upload(bm, U): the complement is stored when the cardinality exceeds U/2
// (src/upload.cpp:296-316).
static int upload_with_universe(const HostContainer* containers, uint32_t n, uint32_t universe_size,
                                cr_stream_t stream, uint32_t bitmap_threshold, cr_gpu_roaring* out)
{
    const uint64_t card = host_cardinality(containers, n);
    if (card > static_cast<uint64_t>(universe_size) / 2u) {  // src/upload.cpp:300-313
        std::vector<std::vector<uint64_t>> storage;
        auto comp = complement_containers(containers, n, universe_size, storage);
        return cr_upload_containers(comp.data(), static_cast<uint32_t>(comp.size()), universe_size, true, card, stream,
                                    bitmap_threshold, out);
    }
    return cr_upload_containers(containers, n, universe_size, false, card, stream, bitmap_threshold, out);
}

GpuRoaring upload(const HostContainer* containers, uint32_t n, uint32_t universe_size, hipStream_t stream,
                  uint32_t bitmap_threshold)
{
    GpuRoaring r;
    throw_on_error(upload_with_universe(containers, n, universe_size, S(stream), bitmap_threshold, to_abi(&r)),
                   "upload");
    return r;
}

// ---- Roaring portable format: host-side parse of the headers ----------------
// Layout (RoaringFormatSpec, little-endian): cookie u32 12346 + u32 size, or
// u16 12347 + u16 size-1 + ceil(size/8) run-flag bytes; size x (u16 key,
// u16 card-1); u32 offsets iff no run container or size >= 4 (not consulted:
// payloads are read in sequence, as CRoaring does); then each payload (run:
// u16 n_runs + (start, length-1) pairs; card <= 4096: u16 values; else 1024 u64).
static uint32_t rd16(const uint8_t* p) { return static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8); }
static uint32_t rd32(const uint8_t* p) { return rd16(p) | (rd16(p + 2) << 16); }

static const char* parse_portable(const uint8_t* buf, size_t len, std::vector<HostContainer>& out,
                                  std::vector<std::vector<uint64_t>>& storage)
{
    out.clear();
    storage.clear();
    if (len < 4) return "truncated cookie";
    const uint32_t c0 = rd32(buf);
    uint32_t n;
    const uint8_t* run_flags = nullptr;
    size_t pos;
    if ((c0 & 0xFFFFu) == 12347u) {
        n = (c0 >> 16) + 1u;
        run_flags = buf + 4;
        pos = 4u + (n + 7u) / 8u;
    } else if (c0 == 12346u) {
        if (len < 8) return "truncated size";
        n = rd32(buf + 4);
        if (n > 65536u) return "more than 65536 containers";
        pos = 8;
    } else {
        return "unknown cookie";
    }
    if (pos + 4ull * n > len) return "truncated header";
    const uint8_t* hdr = buf + pos;
    pos += 4ull * n;
    if (!run_flags || n >= 4u) pos += 4ull * n;
    if (pos > len) return "truncated offset header";
    out.resize(n);
    // payloads that are not 2-byte aligned in `buf` are copied to `storage`
    auto place = [&](size_t at, size_t bytes) -> const void* {
        if ((reinterpret_cast<uintptr_t>(buf + at) & 1u) == 0) return buf + at;
        storage.emplace_back((bytes + 7) / 8);
        std::memcpy(storage.back().data(), buf + at, bytes);
        return storage.back().data();
    };
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t key = rd16(hdr + 4u * i), card = rd16(hdr + 4u * i + 2u) + 1u;
        if (i > 0 && key <= out[i - 1].key) return "keys not strictly increasing";
        HostContainer& h = out[i];
        h.key = static_cast<uint16_t>(key);
        if (run_flags && ((run_flags[i / 8u] >> (i % 8u)) & 1u)) {
            if (pos + 2 > len) return "truncated run container";
            const uint32_t nr = rd16(buf + pos);
            pos += 2;
            if (pos + 4ull * nr > len) return "truncated run container";
            for (uint32_t k = 0; k < nr; ++k)
                if (rd16(buf + pos + 4ull * k) + rd16(buf + pos + 4ull * k + 2) > 0xFFFFu) return "run past 0xFFFF";
            h.typecode = CR_TC_RUN;
            h.cardinality = static_cast<int32_t>(nr);
            h.data = nr ? place(pos, 4ull * nr) : nullptr;
            pos += 4ull * nr;
        } else if (card <= 4096u) {
            if (pos + 2ull * card > len) return "truncated array container";
            h.typecode = CR_TC_ARRAY;
            h.cardinality = static_cast<int32_t>(card);
            h.data = place(pos, 2ull * card);
            pos += 2ull * card;
        } else {
            if (pos + 8192 > len) return "truncated bitset container";
            h.typecode = CR_TC_BITSET;
            h.cardinality = static_cast<int32_t>(card);
            h.data = buf + pos;  // copied with memcpy by the upload
            pos += 8192;
        }
    }
    return nullptr;
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

extern "C" int cr_portable_deserialize(const void* buf, size_t len, uint32_t universe_size, cr_stream_t stream,
                                       uint32_t bitmap_threshold, cr_gpu_roaring* out)
{
    if (!out || (len && !buf)) {
        crimpl::set_error("cr_portable_deserialize: invalid argument");
        return CR_ERR_INVALID;
    }
    std::vector<cu_roaring::HostContainer> conts;
    std::vector<std::vector<uint64_t>> storage;
    const char* err = cu_roaring::parse_portable(static_cast<const uint8_t*>(buf), len, conts, storage);
    if (err) {
        crimpl::set_error("cr_portable_deserialize: %s", err);
        return CR_ERR_INVALID;
    }
    const uint32_t n = static_cast<uint32_t>(conts.size());
    if (universe_size == 0) return cr_upload_containers(conts.data(), n, 0, false, 0, stream, bitmap_threshold, out);
    return cu_roaring::upload_with_universe(conts.data(), n, universe_size, stream, bitmap_threshold, out);
}

namespace cu_roaring {

GpuRoaring portable_deserialize(const void* buf, size_t len, hipStream_t stream, uint32_t bitmap_threshold)
{
    GpuRoaring r;
    throw_on_error(cr_portable_deserialize(buf, len, 0, S(stream), bitmap_threshold, to_abi(&r)), "portable_deserialize");
    return r;
}

GpuRoaring portable_deserialize(const void* buf, size_t len, uint32_t universe_size, hipStream_t stream,
                                uint32_t bitmap_threshold)
{
    GpuRoaring r;
    throw_on_error(cr_portable_deserialize(buf, len, universe_size, S(stream), bitmap_threshold, to_abi(&r)),
                   "portable_deserialize");
    return r;
}

}  // namespace cu_roaring

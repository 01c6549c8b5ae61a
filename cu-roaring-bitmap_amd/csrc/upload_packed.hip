// Packed upload of a host Roaring container list (the reference's upload()).
//
// Layout rules follow src/upload.cpp:89-287 (reference): the universe is the
// explicit one or (last key + 1) << 16 (u32, wraps); AUTO resolves through the
// L2 rule; an effective threshold below 4096 promotes every container, except
// that AUTO skips promotion when n * 16 KiB >= ceil(U/8); container types are
// kept otherwise; cards are u16 (bitset 65536 -> 0, run = n_runs); one device
// allocation holds everything (_alloc_base).
//
// Non-promoted payloads are packed on the host into a pinned buffer and copied
// with one H2D.  When promoting, the raw array/run payloads travel instead and
// a kernel expands them into their 8 KiB bitmap slots through LDS.
#include <algorithm>
#include <cstring>
#include <mutex>
#include <vector>

#include "internal.hpp"

namespace crimpl {

static PinnedStage g_stage;

struct ExpandDesc {
    uint32_t type;     // CR_TC_*
    uint32_t raw_off;  // byte offset of the raw payload in the staging area
    uint32_t card;     // elements (bitset/array) or runs
    uint32_t slot;     // destination bitmap slot
};

__global__ __launch_bounds__(256) void expand_containers(const ExpandDesc* desc, uint32_t n, const uint8_t* raw,
                                                         uint64_t* pool)
{
    __shared__ uint32_t bm[2048];
    const uint32_t t = threadIdx.x;
    for (uint32_t i = blockIdx.x; i < n; i += gridDim.x) {
        const ExpandDesc d = desc[i];
        uint32_t* dst = reinterpret_cast<uint32_t*>(pool) + static_cast<uint64_t>(d.slot) * 2048u;
        if (d.type == CR_TC_BITSET) {
            const uint32_t* src = reinterpret_cast<const uint32_t*>(raw + d.raw_off);
            for (uint32_t k = t; k < 2048u; k += 256) dst[k] = src[k];
            continue;
        }
        for (uint32_t k = t; k < 2048u; k += 256) bm[k] = 0;
        __syncthreads();
        const uint16_t* p = reinterpret_cast<const uint16_t*>(raw + d.raw_off);
        if (d.type == CR_TC_ARRAY) {
            for (uint32_t k0 = t; k0 < d.card; k0 += 8u * 256u) {  // eight values a thread in flight
                uint32_t x[8];
#pragma unroll
                for (uint32_t j = 0; j < 8u; ++j) x[j] = k0 + 256u * j < d.card ? static_cast<uint32_t>(p[k0 + 256u * j]) : ~0u;
#pragma unroll
                for (uint32_t j = 0; j < 8u; ++j)
                    if (x[j] != ~0u) atomicOr(&bm[x[j] >> 5], 1u << (x[j] & 31u));
            }
        } else {
            for (uint32_t r = t; r < d.card; r += 256) {  // [start, start+len], src/upload.cpp:194-197
                const uint32_t s = p[2 * r];
                uint32_t e = s + p[2 * r + 1];
                if (e > 0xFFFFu) e = 0xFFFFu;
                const uint32_t ws = s >> 5, we = e >> 5;
                const uint32_t ms = ~0u << (s & 31u), me = ~0u >> (31u - (e & 31u));
                if (ws == we) {
                    atomicOr(&bm[ws], ms & me);
                } else {
                    atomicOr(&bm[ws], ms);
                    for (uint32_t w = ws + 1; w < we; ++w) bm[w] = ~0u;
                    atomicOr(&bm[we], me);
                }
            }
        }
        __syncthreads();
        for (uint32_t k = t; k < 2048u; k += 256) dst[k] = bm[k];
        __syncthreads();
    }
}

static size_t payload_bytes(const cr_host_container& c)
{
    if (c.typecode == CR_TC_BITSET) return 8192;
    if (c.typecode == CR_TC_ARRAY) return static_cast<size_t>(c.cardinality) * 2u;
    return static_cast<size_t>(c.cardinality) * 4u;
}

static uint64_t container_card(const cr_host_container& c)
{
    if (c.typecode != CR_TC_RUN) return static_cast<uint64_t>(c.cardinality);
    const uint16_t* r = static_cast<const uint16_t*>(c.data);
    uint64_t t = 0;
    for (int32_t k = 0; k < c.cardinality; ++k) t += static_cast<uint64_t>(r[2 * k + 1]) + 1u;
    return t;
}

int upload_containers_impl(const cr_host_container* conts, uint32_t n, uint32_t explicit_u, bool complemented,
                           uint64_t logical, hipStream_t s, uint32_t thr, cr_gpu_roaring* out)
{
    reset(out);
    if (n == 0) {  // src/upload.cpp:268-272
        out->universe_size = explicit_u;
        if (complemented) {
            out->negated = true;
            out->total_cardinality = logical;
        }
        return CR_OK;
    }
    for (uint32_t i = 0; i < n; ++i) {
        const cr_host_container& c = conts[i];
        const bool bad_type = c.typecode != CR_TC_BITSET && c.typecode != CR_TC_ARRAY && c.typecode != CR_TC_RUN;
        if (bad_type || c.cardinality < 0 || (i > 0 && conts[i - 1].key >= c.key) ||
            (c.cardinality > 0 && c.data == nullptr)) {
            set_error("cr_upload_containers: container %u is malformed (type, order, or payload)", i);
            return CR_ERR_INVALID;
        }
    }
    uint32_t universe = explicit_u;
    if (universe == 0) universe = (static_cast<uint32_t>(conts[n - 1].key) + 1u) << 16;  // :96-100
    const uint32_t eff = thr == CR_PROMOTE_AUTO ? resolve_auto_threshold(universe, -1) : thr;
    bool promote = eff < CR_PROMOTE_KEEP_DEFAULT;  // :104
    if (promote && thr == CR_PROMOTE_AUTO) {       // :112-118
        const uint64_t promoted = static_cast<uint64_t>(n) * 1024u * 8u;
        const uint64_t bitset = (static_cast<uint64_t>(universe) + 7u) / 8u;
        if (promoted * 2u >= bitset) promote = false;
    }
    uint64_t bmp_words = 0, arr_elems = 0, run_pairs = 0, raw_bytes = 0;
    uint32_t nb = 0, na = 0, nr = 0;
    for (uint32_t i = 0; i < n; ++i) {
        const cr_host_container& c = conts[i];
        if (c.typecode == CR_TC_BITSET || promote) {
            ++nb;
            bmp_words += 1024;
        } else if (c.typecode == CR_TC_ARRAY) {
            ++na;
            arr_elems += static_cast<uint64_t>(c.cardinality);
        } else {
            ++nr;
            run_pairs += static_cast<uint64_t>(c.cardinality);
        }
        raw_bytes += (payload_bytes(c) + 3u) & ~size_t(3);
    }
    const uint32_t max_key = conts[n - 1].key;
    const uint64_t kidx_len = static_cast<uint64_t>(max_key) + 1u;
    const OutLayout L = plan_out(n, kidx_len, bmp_words, arr_elems, run_pairs * 2u);
    CR_RET(alloc_out(out, L, n, kidx_len, bmp_words, arr_elems, run_pairs * 2u, s));

    // Host staging mirrors the device block (metadata + pools); when promoting the
    // bitmap section is produced on the device and the raw payloads follow.
    const size_t raw_off0 = (L.total + 255) & ~size_t(255);
    const size_t desc_off = raw_off0 + ((raw_bytes + 255) & ~size_t(255));
    const size_t stage_bytes = promote ? desc_off + sizeof(ExpandDesc) * n : L.total;
    std::lock_guard<std::mutex> lock(g_stage.mu);
    CR_RET(g_stage.reserve(stage_bytes));
    char* h = static_cast<char*>(g_stage.ptr);
    auto* keys = reinterpret_cast<uint16_t*>(h + L.keys);
    auto* types = reinterpret_cast<uint8_t*>(h + L.types);
    auto* offs = reinterpret_cast<uint32_t*>(h + L.offsets);
    auto* cards = reinterpret_cast<uint16_t*>(h + L.cards);
    auto* kidx = reinterpret_cast<uint16_t*>(h + L.kidx);
    auto* bmp = reinterpret_cast<uint64_t*>(h + L.bmp);
    auto* arr = reinterpret_cast<uint16_t*>(h + L.arr);
    auto* run = reinterpret_cast<uint16_t*>(h + L.run);
    auto* desc = reinterpret_cast<ExpandDesc*>(h + desc_off);
    std::memset(kidx, 0xFF, kidx_len * 2u);
    uint64_t bc = 0, ac = 0, rc = 0, rawc = 0, total = 0;
    for (uint32_t i = 0; i < n; ++i) {  // pack_into_buffer, :155-225
        const cr_host_container& c = conts[i];
        keys[i] = c.key;
        kidx[c.key] = static_cast<uint16_t>(i);
        total += container_card(c);
        const uint32_t card = static_cast<uint32_t>(c.cardinality);
        cards[i] = static_cast<uint16_t>(c.typecode == CR_TC_BITSET && card > 65535u ? 0u : card);
        if (promote || c.typecode == CR_TC_BITSET) {
            types[i] = CR_BITMAP;
            offs[i] = static_cast<uint32_t>(bc * 8u);
            if (promote) {
                const size_t pb = payload_bytes(c);
                std::memcpy(h + raw_off0 + rawc, c.data, pb);
                desc[i] = ExpandDesc{c.typecode, static_cast<uint32_t>(rawc), card, static_cast<uint32_t>(bc / 1024u)};
                rawc += (pb + 3u) & ~size_t(3);
            } else {
                std::memcpy(bmp + bc, c.data, 8192);
            }
            bc += 1024;
        } else if (c.typecode == CR_TC_ARRAY) {
            types[i] = CR_ARRAY;
            offs[i] = static_cast<uint32_t>(ac * 2u);
            std::memcpy(arr + ac, c.data, static_cast<size_t>(card) * 2u);
            ac += card;
        } else {
            types[i] = CR_RUN;
            offs[i] = static_cast<uint32_t>(rc * 4u);
            std::memcpy(run + rc * 2u, c.data, static_cast<size_t>(card) * 4u);
            rc += card;
        }
    }
    char* d = static_cast<char*>(out->_alloc_base);
    if (!promote) {
        CR_HIP_RET(hipMemcpyAsync(d, h, L.total, hipMemcpyHostToDevice, s));
    } else {
        // metadata sections (everything after the bitmap pool), then raw payloads
        const size_t meta_lo = L.keys;
        CR_HIP_RET(hipMemcpyAsync(d + meta_lo, h + meta_lo, L.total - meta_lo, hipMemcpyHostToDevice, s));
        Scratch raw;
        CR_RET(raw.alloc(stage_bytes - raw_off0, s));
        CR_HIP_RET(hipMemcpyAsync(raw.ptr, h + raw_off0, stage_bytes - raw_off0, hipMemcpyHostToDevice, s));
        const ExpandDesc* ddesc = raw.at<ExpandDesc>(desc_off - raw_off0);
        {
            CR_TIMED("expand_containers", s);
            expand_containers<<<std::min<uint32_t>(n, 4096u), 256, 0, s>>>(ddesc, n, raw.at<uint8_t>(0),
                                                                            out->bitmap_data);
        }
        CR_LAUNCH_CHECK();
        CR_RET(sync_stream(s));
    }
    CR_RET(sync_stream(s));  // the staging buffer is reused by the next call
    out->n_containers = n;
    out->n_bitmap_containers = nb;
    out->n_array_containers = na;
    out->n_run_containers = nr;
    out->universe_size = universe;
    out->total_cardinality = complemented ? logical : total;
    out->negated = complemented;
    out->max_key = max_key;
    out->array_pool_bytes = static_cast<uint32_t>(arr_elems * 2u);
    out->run_pool_bytes = static_cast<uint32_t>(run_pairs * 4u);
    if (arr_elems == 0) out->array_data = nullptr;
    if (run_pairs == 0) out->run_data = nullptr;
    if (bmp_words == 0) out->bitmap_data = nullptr;
    return CR_OK;
}

}  // namespace crimpl

using namespace crimpl;

extern "C" int cr_upload_containers(const cr_host_container* containers, uint32_t n, uint32_t universe_size,
                                    bool complemented, uint64_t logical_cardinality, cr_stream_t stream,
                                    uint32_t bitmap_threshold, cr_gpu_roaring* out)
{
    if (!out || (n && !containers)) {
        set_error("cr_upload_containers: invalid argument");
        return CR_ERR_INVALID;
    }
    reset(out);
    return produced(upload_containers_impl(containers, n, universe_size, complemented, logical_cardinality,
                                           as_stream(stream), bitmap_threshold, out),
                    out, as_stream(stream));
}

extern "C" int cr_get_meta(const cr_host_container* c, uint32_t n, cr_meta* out)
{
    if (!out || (n && !c)) {
        set_error("cr_get_meta: invalid argument");
        return CR_ERR_INVALID;
    }
    std::memset(out, 0, sizeof(*out));  // src/upload.cpp:31-71
    out->n_containers = n;
    size_t arr = 0, runs = 0;
    for (uint32_t i = 0; i < n; ++i) {
        if (c[i].typecode == CR_TC_BITSET) {
            ++out->n_bitmap_containers;
        } else if (c[i].typecode == CR_TC_ARRAY) {
            ++out->n_array_containers;
            arr += static_cast<size_t>(c[i].cardinality);
        } else if (c[i].typecode == CR_TC_RUN) {
            ++out->n_run_containers;
            runs += static_cast<size_t>(c[i].cardinality);
        }
    }
    if (n > 0) out->universe_size = (static_cast<uint32_t>(c[n - 1].key) + 1u) << 16;
    out->total_bytes = n * (2u + 1u + 4u + 2u) + static_cast<size_t>(out->n_bitmap_containers) * 8192u + arr * 2u +
                       runs * 4u;
    return CR_OK;
}

// GpuRoaring -> the Roaring portable format, on the device.
//
// The portable format (the layout CRoaring's roaring_bitmap_portable_serialize
// writes; no counterpart in the reference, whose bench_from_disk reads such
// files, bench/CMakeLists.txt:89-93) has no complement flag, so the logical set
// is written: a negated bitmap is complemented within [0, U) key by key.
// Every output container is re-encoded from its logical image by CRoaring's
// run_optimize rule: array if cardinality <= 4096, else bitset, unless the run
// encoding (2 + 4 n_runs bytes) is smaller than that (2 + 2 card, or 8192).
// Empty containers (a set-operation result may hold them) are not written.
//
// Two passes over candidate keys (the containers, or every key below
// ceil(U / 65536) when negated), one workgroup each, each building the
// container's logical image in LDS:
//   ps_plan   cardinality, run count, encoding and payload bytes;
//   ps_write  the payload, into a device staging buffer at its scanned offset.
// The host then assembles the small header (cookie, run flags, key/card pairs,
// offsets) from the plan and copies the payloads behind it.
#include <algorithm>
#include <cstring>
#include <vector>

#include "image.hpp"
#include "internal.hpp"

namespace crimpl {

namespace {

constexpr uint8_t PS_NONE = 0, PS_ARRAY = 1, PS_BITMAP = 2, PS_RUN = 3;

struct PsPlan {
    uint16_t* key;
    uint32_t* card;
    uint8_t* form;
    uint64_t* bytes;  // payload bytes (scanned into offsets)
    uint32_t* any_run;
};

// Logical image of candidate i into img.w; returns the candidate's key.
__device__ uint32_t ps_image(const cr_gpu_roaring& r, uint32_t i, Image* img, int32_t* s_c)
{
    const uint32_t t = threadIdx.x;
    const bool neg = r.negated;
    uint32_t key;
    if (!neg) {
        key = r.keys[i];
        if (t == 0) *s_c = static_cast<int32_t>(i);
    } else {
        key = i;
        if (r.key_index && key <= r.max_key) {
            if (t == 0) {
                const uint16_t e = r.key_index[key];
                *s_c = e == 0xFFFFu ? -1 : static_cast<int32_t>(e);
            }
        } else if (t < 64) {
            const uint32_t pos = wave_lower_bound_u16(r.keys, r.n_containers, key);
            if (t == 0) *s_c = (pos < r.n_containers && r.keys[pos] == key) ? static_cast<int32_t>(pos) : -1;
        }
    }
    __syncthreads();
    const int32_t c = *s_c;
    const uint8_t type = c >= 0 ? r.types[c] : 0xFFu;
    if (type == CR_BITMAP) {
        const uint32_t* src = reinterpret_cast<const uint32_t*>(r.bitmap_data + r.offsets[c] / 8u);
        if ((reinterpret_cast<uintptr_t>(src) & 15u) == 0) {
            const uint4* s4 = reinterpret_cast<const uint4*>(src);
            uint4 v[2];
#pragma unroll
            // Ordinary loads: ps_plan's read keeps the payload in the Infinity
            // Cache for ps_write's (60 -> 55 us on 16384 bitmaps).
            for (int j = 0; j < 2; ++j) v[j] = s4[j * CV_NT + t];
#pragma unroll
            for (int j = 0; j < 2; ++j) reinterpret_cast<uint4*>(img->w)[j * CV_NT + t] = v[j];
        } else {
#pragma unroll
            for (int j = 0; j < CV_WPT; ++j) img->w[j * CV_NT + t] = src[j * CV_NT + t];
        }
        __syncthreads();
    } else if (type == CR_ARRAY) {
        expand_to_lds(CR_ARRAY, r.array_data + r.offsets[c] / 2u, r.cardinalities[c], img);
    } else if (type == CR_RUN) {
        expand_to_lds(CR_RUN, r.run_data + r.offsets[c] / 2u, r.cardinalities[c], img);
    } else {
#pragma unroll
        for (int j = 0; j < CV_WPT; ++j) img->w[j * CV_NT + t] = 0;
        __syncthreads();
    }
    if (neg) {  // complement within [0, U): bits of this key below U - key * 65536
        const uint64_t lo = static_cast<uint64_t>(key) << 16;
        const uint64_t rest = r.universe_size > lo ? r.universe_size - lo : 0u;
        const uint64_t valid = rest < 65536u ? rest : 65536u;
#pragma unroll
        for (int j = 0; j < CV_WPT; ++j) {
            const uint32_t w = j * CV_NT + t;
            const uint64_t b0 = 32ull * w;
            uint32_t m = 0;
            if (b0 + 32u <= valid)
                m = ~0u;
            else if (b0 < valid)
                m = (1u << (valid - b0)) - 1u;
            img->w[w] = ~img->w[w] & m;
        }
        __syncthreads();
    }
    return key;
}

// Run starts / ends of word j (of thread t's eight words [8t, 8t + 8)).
__device__ __forceinline__ uint32_t starts_of(const uint32_t* w, uint32_t i)
{
    const uint32_t prev = i ? w[i - 1] >> 31 : 0u;
    return w[i] & ~((w[i] << 1) | prev);
}
__device__ __forceinline__ uint32_t ends_of(const uint32_t* w, uint32_t i)
{
    const uint32_t next = i + 1 < 2048u ? (w[i + 1] & 1u) << 31 : 0u;
    return w[i] & ~((w[i] >> 1) | next);
}

__device__ __forceinline__ uint8_t ps_choose(uint32_t card, uint32_t nr, uint64_t* bytes)
{
    if (card == 0) {
        *bytes = 0;
        return PS_NONE;
    }
    const uint32_t run_size = 2u + 4u * nr;
    const bool is_array = card <= 4096u;
    const uint32_t cur = is_array ? 2u + 2u * card : 8192u;
    if (run_size < cur) {
        *bytes = run_size;
        return PS_RUN;
    }
    *bytes = is_array ? 2ull * card : 8192u;
    return is_array ? PS_ARRAY : PS_BITMAP;
}

__global__ __launch_bounds__(CV_NT) void ps_plan(cr_gpu_roaring r, PsPlan p)
{
    __shared__ Image img;
    __shared__ int32_t s_c;
    __shared__ uint32_t red[CV_NT / 64];
    const uint32_t i = blockIdx.x;
    const uint32_t t = threadIdx.x;
    const uint32_t key = ps_image(r, i, &img, &s_c);
    uint32_t card = 0, nr = 0;
#pragma unroll
    for (int j = 0; j < CV_WPT; ++j) {
        const uint32_t w = CV_WPT * t + j;
        card += __popc(img.w[w]);
        nr += __popc(starts_of(img.w, w));
    }
    card = block_sum<CV_NT>(card, red);
    nr = block_sum<CV_NT>(nr, red);
    if (t == 0) {
        uint64_t bytes;
        const uint8_t form = ps_choose(card, nr, &bytes);
        p.key[i] = static_cast<uint16_t>(key);
        p.card[i] = card;
        p.form[i] = form;
        p.bytes[i] = bytes;
        if (form == PS_RUN) atomicOr(p.any_run, 1u);
    }
}

__device__ __forceinline__ void put_u16(uint8_t* base, uint64_t byte_off, uint32_t v)
{
    *reinterpret_cast<uint16_t*>(base + byte_off) = static_cast<uint16_t>(v);
}

__global__ __launch_bounds__(CV_NT) void ps_write(cr_gpu_roaring r, const uint8_t* form_of, const uint64_t* offset_of,
                                                  uint8_t* __restrict__ out)
{
    __shared__ Image img;
    __shared__ uint16_t stage[2 * 4096];  // array values, or run (start, end) pairs
    __shared__ int32_t s_c;
    __shared__ uint32_t red[CV_NT / 64];
    const uint32_t i = blockIdx.x;
    const uint32_t t = threadIdx.x;
    const uint8_t form = form_of[i];
    if (form == PS_NONE) return;
    ps_image(r, i, &img, &s_c);
    const uint64_t off = offset_of[i];
    if (form == PS_BITMAP) {
        if ((off & 15u) == 0) {
            uint4* d = reinterpret_cast<uint4*>(out + off);
            const uint4* s4 = reinterpret_cast<const uint4*>(img.w);
#pragma unroll
            for (int j = 0; j < 2; ++j) st_stream(d + j * CV_NT + t, s4[j * CV_NT + t]);
        } else if ((off & 3u) == 0) {
            uint32_t* d = reinterpret_cast<uint32_t*>(out + off);
#pragma unroll
            for (int j = 0; j < CV_WPT; ++j) d[j * CV_NT + t] = img.w[j * CV_NT + t];
        } else {
            for (uint32_t k = t; k < 4096u; k += CV_NT) put_u16(out, off + 2ull * k, img.w[k >> 1] >> (16u * (k & 1u)));
        }
        return;
    }
    if (form == PS_ARRAY) {
        uint32_t n = 0;
#pragma unroll
        for (int j = 0; j < CV_WPT; ++j) n += __popc(img.w[CV_WPT * t + j]);
        uint32_t total;
        uint32_t pos = block_excl_scan<CV_NT>(n, red, total);
#pragma unroll
        for (int j = 0; j < CV_WPT; ++j) {
            const uint32_t w = CV_WPT * t + j;
            for (uint32_t x = img.w[w]; x; x &= x - 1) stage[pos++] = static_cast<uint16_t>(32u * w + __builtin_ctz(x));
        }
        __syncthreads();
        for (uint32_t k = t; k < total; k += CV_NT) put_u16(out, off + 2ull * k, stage[k]);
        return;
    }
    // PS_RUN: the k-th start bit pairs with the k-th end bit
    uint32_t ns = 0, ne = 0;
#pragma unroll
    for (int j = 0; j < CV_WPT; ++j) {
        ns += __popc(starts_of(img.w, CV_WPT * t + j));
        ne += __popc(ends_of(img.w, CV_WPT * t + j));
    }
    uint32_t nr, nr2;
    uint32_t ps = block_excl_scan<CV_NT>(ns, red, nr);
    uint32_t pe = block_excl_scan<CV_NT>(ne, red, nr2);
#pragma unroll
    for (int j = 0; j < CV_WPT; ++j) {
        const uint32_t w = CV_WPT * t + j;
        for (uint32_t x = starts_of(img.w, w); x; x &= x - 1) stage[2 * ps++] = static_cast<uint16_t>(32u * w + __builtin_ctz(x));
        for (uint32_t x = ends_of(img.w, w); x; x &= x - 1) stage[2 * pe++ + 1] = static_cast<uint16_t>(32u * w + __builtin_ctz(x));
    }
    __syncthreads();
    if (t == 0) put_u16(out, off, nr);
    for (uint32_t k = t; k < nr; k += CV_NT) {
        put_u16(out, off + 2u + 4ull * k, stage[2 * k]);
        put_u16(out, off + 4u + 4ull * k, static_cast<uint32_t>(stage[2 * k + 1]) - stage[2 * k]);
    }
}

// Plan + scans; fills the host copy of the plan and the serialized size.
struct HostPlan {
    uint32_t n_cand = 0, n_out = 0;
    bool any_run = false;
    uint64_t payload = 0, header = 0;
    std::vector<uint16_t> key;
    std::vector<uint32_t> card;
    std::vector<uint8_t> form;
    std::vector<uint64_t> offset;  // payload offset within the payload region
};

uint32_t candidates(const cr_gpu_roaring* bm)
{
    if (!bm->negated) return bm->n_containers;
    return static_cast<uint32_t>((static_cast<uint64_t>(bm->universe_size) + 65535u) >> 16);
}

uint64_t header_bytes(uint32_t n, bool any_run)
{
    uint64_t h = any_run ? 4u + (n + 7u) / 8u : 8u;
    h += 4ull * n;
    if (!any_run || n >= 4u) h += 4ull * n;
    return h;
}

int plan_portable(const cr_gpu_roaring* bm, hipStream_t s, Scratch& sc, HostPlan& hp, PsPlan& p, uint64_t*& offs)
{
    const uint32_t K = candidates(bm);
    hp.n_cand = K;
    if (K == 0) {
        hp.header = header_bytes(0, false);
        return CR_OK;
    }
    Carver cv;
    const size_t o_key = cv.add(K * 2ull), o_card = cv.add(K * 4ull), o_form = cv.add(K), o_bytes = cv.add(K * 8ull),
                 o_offs = cv.add(K * 8ull), o_any = cv.add(4);
    CR_RET(sc.alloc(cv.total, s));
    p = PsPlan{sc.at<uint16_t>(o_key), sc.at<uint32_t>(o_card), sc.at<uint8_t>(o_form), sc.at<uint64_t>(o_bytes),
               sc.at<uint32_t>(o_any)};
    offs = sc.at<uint64_t>(o_offs);
    CR_RET(fill_u32(p.any_run, 0u, 1, s));
    {
        CR_TIMED("ps_plan", s);
        ps_plan<<<K, CV_NT, 0, s>>>(*bm, p);
    }
    CR_LAUNCH_CHECK();
    CR_RET(scan_exclusive_u64(p.bytes, K, offs, s));
    hp.key.resize(K);
    hp.card.resize(K);
    hp.form.resize(K);
    hp.offset.resize(K);
    std::vector<uint64_t> bytes(K);
    uint32_t any = 0;
    CR_HIP_RET(hipMemcpyAsync(hp.key.data(), p.key, K * 2ull, hipMemcpyDeviceToHost, s));
    CR_HIP_RET(hipMemcpyAsync(hp.card.data(), p.card, K * 4ull, hipMemcpyDeviceToHost, s));
    CR_HIP_RET(hipMemcpyAsync(hp.form.data(), p.form, K, hipMemcpyDeviceToHost, s));
    CR_HIP_RET(hipMemcpyAsync(hp.offset.data(), offs, K * 8ull, hipMemcpyDeviceToHost, s));
    CR_HIP_RET(hipMemcpyAsync(bytes.data(), p.bytes, K * 8ull, hipMemcpyDeviceToHost, s));
    CR_HIP_RET(hipMemcpyAsync(&any, p.any_run, 4, hipMemcpyDeviceToHost, s));
    CR_RET(sync_stream(s));
    for (uint32_t i = 0; i < K; ++i) hp.n_out += hp.form[i] != PS_NONE;
    hp.any_run = any != 0;
    hp.payload = hp.offset[K - 1] + bytes[K - 1];
    hp.header = header_bytes(hp.n_out, hp.any_run);
    return CR_OK;
}

// Device -> pageable host memory through two pinned 32 MiB chunks: the DMA of
// one chunk overlaps the host copy of the previous one (a direct copy into
// pageable memory runs at a fraction of the link rate).
PinnedStage g_ser_stage;

int copy_to_host(uint8_t* dst, const uint8_t* src, uint64_t bytes, hipStream_t s)
{
    constexpr uint64_t CH = 32ull << 20;
    std::lock_guard<std::mutex> lock(g_ser_stage.mu);
    CR_RET(g_ser_stage.reserve(2 * CH));
    uint8_t* pin = static_cast<uint8_t*>(g_ser_stage.ptr);
    hipEvent_t ev[2] = {nullptr, nullptr};
    for (int i = 0; i < 2; ++i) CR_HIP_RET(hipEventCreateWithFlags(&ev[i], hipEventDisableTiming));
    const uint64_t n = (bytes + CH - 1) / CH;
    auto drain = [&](uint64_t i) -> hipError_t {  // chunk i has landed in its pinned half: copy it out
        const hipError_t e = hipEventSynchronize(ev[i & 1]);
        if (e == hipSuccess) std::memcpy(dst + i * CH, pin + (i & 1) * CH, std::min(CH, bytes - i * CH));
        return e;
    };
    hipError_t e = hipSuccess;
    for (uint64_t i = 0; i < n && e == hipSuccess; ++i) {
        if (i >= 2) e = drain(i - 2);
        if (e == hipSuccess)
            e = hipMemcpyAsync(pin + (i & 1) * CH, src + i * CH, std::min(CH, bytes - i * CH), hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipEventRecord(ev[i & 1], s);
    }
    for (uint64_t i = n > 2 ? n - 2 : 0; i < n && e == hipSuccess; ++i) e = drain(i);
    for (int i = 0; i < 2; ++i) (void)hipEventDestroy(ev[i]);
    if (e != hipSuccess) {
        set_error("cr_portable_serialize: %s", hipGetErrorString(e));
        return CR_ERR_HIP;
    }
    return CR_OK;
}

void put16h(uint8_t* p, uint32_t v)
{
    p[0] = static_cast<uint8_t>(v);
    p[1] = static_cast<uint8_t>(v >> 8);
}
void put32h(uint8_t* p, uint32_t v)
{
    put16h(p, v & 0xFFFFu);
    put16h(p + 2, v >> 16);
}

}  // namespace
}  // namespace crimpl

using namespace crimpl;

extern "C" int cr_portable_size_in_bytes(const cr_gpu_roaring* bm, cr_stream_t stream, size_t* out_bytes)
{
    if (!bm || !out_bytes) {
        set_error("cr_portable_size_in_bytes: invalid argument");
        return CR_ERR_INVALID;
    }
    hipStream_t s = as_stream(stream);
    Scratch sc;
    HostPlan hp;
    PsPlan p{};
    uint64_t* offs = nullptr;
    CR_RET(plan_portable(bm, s, sc, hp, p, offs));
    *out_bytes = hp.header + hp.payload;
    return CR_OK;
}

extern "C" int cr_portable_serialize(const cr_gpu_roaring* bm, cr_stream_t stream, void* host_buf, size_t capacity,
                                     size_t* written)
{
    if (!bm || !written || (capacity && !host_buf)) {
        set_error("cr_portable_serialize: invalid argument");
        return CR_ERR_INVALID;
    }
    hipStream_t s = as_stream(stream);
    Scratch sc;
    HostPlan hp;
    PsPlan p{};
    uint64_t* offs = nullptr;
    CR_RET(plan_portable(bm, s, sc, hp, p, offs));
    const uint64_t total = hp.header + hp.payload;
    *written = total;
    if (total > capacity) {
        set_error("cr_portable_serialize: buffer of %zu bytes, %llu needed", capacity,
                  static_cast<unsigned long long>(total));
        return CR_ERR_INVALID;
    }
    if (total > 0xFFFFFFFFull) {  // offsets are u32
        set_error("cr_portable_serialize: %llu bytes exceed the format's 32-bit offsets",
                  static_cast<unsigned long long>(total));
        return CR_ERR_UNSUPPORTED;
    }
    uint8_t* h = static_cast<uint8_t*>(host_buf);
    const uint32_t n = hp.n_out;
    uint8_t* q = h;
    if (hp.any_run) {
        put16h(q, 12347u);
        put16h(q + 2, n - 1u);
        q += 4;
        std::memset(q, 0, (n + 7u) / 8u);
        uint32_t j = 0;
        for (uint32_t i = 0; i < hp.n_cand; ++i) {
            if (hp.form[i] == PS_NONE) continue;
            if (hp.form[i] == PS_RUN) q[j / 8u] |= static_cast<uint8_t>(1u << (j % 8u));
            ++j;
        }
        q += (n + 7u) / 8u;
    } else {
        put32h(q, 12346u);
        put32h(q + 4, n);
        q += 8;
    }
    for (uint32_t i = 0; i < hp.n_cand; ++i) {
        if (hp.form[i] == PS_NONE) continue;
        put16h(q, hp.key[i]);
        put16h(q + 2, hp.card[i] - 1u);
        q += 4;
    }
    if (!hp.any_run || n >= 4u) {
        for (uint32_t i = 0; i < hp.n_cand; ++i) {
            if (hp.form[i] == PS_NONE) continue;
            put32h(q, static_cast<uint32_t>(hp.header + hp.offset[i]));
            q += 4;
        }
    }
    if (hp.payload == 0) return CR_OK;
    void* stage = nullptr;
    CR_RET(dev_alloc(&stage, hp.payload, s));
    {
        CR_TIMED("ps_write", s);
        ps_write<<<hp.n_cand, CV_NT, 0, s>>>(*bm, p.form, offs, static_cast<uint8_t*>(stage));
    }
    hipError_t e = hipGetLastError();
    int rc = e == hipSuccess ? copy_to_host(h + hp.header, static_cast<const uint8_t*>(stage), hp.payload, s)
                             : CR_ERR_HIP;
    if (e != hipSuccess) set_error("cr_portable_serialize: %s", hipGetErrorString(e));
    dev_free(stage, s);
    return rc;
}

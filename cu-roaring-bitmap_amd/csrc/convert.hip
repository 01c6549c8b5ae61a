// Conversions of a GpuRoaring: decompress_to_bitset, enumerate_ids,
// promote_to_bitmap / promote_auto and the deep copy.
//
// Output semantics follow the reference (src/decompress.cu:104-162,
// src/to_csr.cu:161-220, src/promote.cu:178-385).  None of these calls
// synchronises its stream (the reference's contract for them).

#include <algorithm>
#include <cstring>
#include <mutex>
#include <type_traits>

#include "image.hpp"
#include "internal.hpp"

namespace crimpl {

namespace {

// ---- decompress_to_bitset ---------------------------------------------------
// One workgroup per 2048-word key region of the output: the region is written
// once (the container's bits, zeros when the key is absent), and the
// complement of a negated bitmap is applied on the way out (words below U/32
// inverted, the tail word's valid bits flipped, src/decompress.cu:128-150).
// Writes stay below n_words.
// LEAN: one wavefront per region and no run difference array (inputs that
// hold no run container), so more regions are in flight per CU.
template <int NT, bool LEAN>
__global__ __launch_bounds__(NT) void cv_decompress(cr_gpu_roaring r, uint32_t* __restrict__ out, uint32_t n_words)
{
    constexpr int WPT = 2048 / NT;
    __shared__ alignas(16) uint32_t w[2048];
    __shared__ int32_t cover[LEAN ? 1 : 2048];
    __shared__ int32_t s_c;
    const uint32_t key = blockIdx.x;
    const uint32_t t = threadIdx.x;
    if (r.key_index && key <= r.max_key) {  // one load through the key index
        if (t == 0) {
            const uint16_t e = r.key_index[key];
            s_c = e == 0xFFFFu ? -1 : static_cast<int32_t>(e);
        }
    } else if (t < 64) {
        const uint32_t pos = wave_lower_bound_u16(r.keys, r.n_containers, key);
        if (t == 0) s_c = (pos < r.n_containers && r.keys[pos] == key) ? static_cast<int32_t>(pos) : -1;
    }
    __syncthreads();
    const int32_t c = s_c;
    const uint8_t type = c >= 0 ? r.types[c] : 0xFFu;
    const uint32_t* src;
    if (type == CR_BITMAP) {
        src = reinterpret_cast<const uint32_t*>(r.bitmap_data + r.offsets[c] / 8u);
    } else {
        if (type == CR_ARRAY || type == CR_RUN) {
            expand_img<NT>(type, (type == CR_ARRAY ? r.array_data : r.run_data) + r.offsets[c] / 2u,
                           r.cardinalities[c], w, LEAN ? nullptr : cover);
        } else {
#pragma unroll
            for (int j = 0; j < WPT; ++j) w[j * NT + t] = 0;
            __syncthreads();
        }
        src = w;
    }
    const uint64_t w0 = static_cast<uint64_t>(key) * 2048u;
    const uint32_t full = r.universe_size / 32u, tail = r.universe_size % 32u;
    const bool neg = r.negated;
    uint32_t* dst = out + w0;
    const bool vec = w0 + 2048u <= n_words &&
                     ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15u) == 0;
    if (vec && (!neg || w0 + 2048u <= full)) {
        constexpr int V = 512 / NT;  // 16-byte words per thread
        uint4* d4 = reinterpret_cast<uint4*>(dst);
        uint4 v[V];
        if (type == CR_BITMAP) {
            const uint4* s4 = reinterpret_cast<const uint4*>(src);
#pragma unroll
            for (int j = 0; j < V; ++j) v[j] = ld_stream(s4 + j * NT + t);
        } else {
            const uint4* l4 = reinterpret_cast<const uint4*>(w);
#pragma unroll
            for (int j = 0; j < V; ++j) v[j] = l4[j * NT + t];
        }
#pragma unroll
        for (int j = 0; j < V; ++j) {
            if (neg) v[j] = make_uint4(~v[j].x, ~v[j].y, ~v[j].z, ~v[j].w);
            st_stream(d4 + j * NT + t, v[j]);
        }
        return;
    }
    for (uint32_t i = t; i < 2048u; i += NT) {
        const uint64_t wd = w0 + i;
        if (wd >= n_words) break;
        uint32_t v = src[i];
        if (neg) {
            if (wd < full)
                v = ~v;
            else if (wd == full && tail)
                v ^= (1u << tail) - 1u;
        }
        dst[i] = v;
    }
}

// ---- enumerate_ids ----------------------------------------------------------
// Per-container id counts (a bitmap's popcount: the reference takes the stored
// cardinality, which reads 0 for a full container), one exclusive scan, then
// one workgroup per container writes its ids in order.  Bitmap and run
// containers go through LDS: the low 16 bits of each 512-word chunk's ids are
// staged in order and then written out as coalesced int64 stores.
// Writes stay below `cap` ids.
// Ids stored in container c (a wave computes it; every lane returns the sum):
// a bitmap's popcount (8 loads of 16 B per lane in flight), an array's
// cardinality, a run container's sum of (length + 1).
__device__ inline uint32_t container_count(const cr_gpu_roaring& r, uint32_t c, uint32_t lane)
{
    const uint8_t type = r.types[c];
    const uint32_t off = r.offsets[c];
    uint32_t n = 0;
    if (type == CR_BITMAP) {
        const uint64_t* p = r.bitmap_data + off / 8u;
        if ((reinterpret_cast<uintptr_t>(p) & 15u) == 0) {
            // 8 KiB = 64 lanes x 8 loads of 16 bytes, all in flight together
            const uint4* bm = reinterpret_cast<const uint4*>(p);
            uint4 v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = ld_stream(bm + j * 64 + lane);
#pragma unroll
            for (int j = 0; j < 8; ++j) n += __popc(v[j].x) + __popc(v[j].y) + __popc(v[j].z) + __popc(v[j].w);
        } else {
            for (uint32_t w = lane; w < 1024u; w += 64) n += static_cast<uint32_t>(__popcll(p[w]));
        }
    } else if (type == CR_ARRAY) {
        n = lane == 0 ? r.cardinalities[c] : 0u;
    } else if (type == CR_RUN) {
        const uint16_t* runs = r.run_data + off / 2u;
        for (uint32_t k = lane; k < r.cardinalities[c]; k += 64) n += static_cast<uint32_t>(runs[2 * k + 1]) + 1u;
    }
    return wave_sum(n);
}

__global__ __launch_bounds__(CV_NT) void cv_enum_count(cr_gpu_roaring r, uint64_t* counts)
{
    const uint32_t c = (blockIdx.x * CV_NT + threadIdx.x) >> 6;
    const uint32_t lane = __lane_id();
    if (c >= r.n_containers) return;
    const uint32_t n = container_count(r, c, lane);
    if (lane == 0) counts[c] = n;
}

// Sum of the containers' counts into *total (zeroed by the caller's stream
// order).  Each wave takes containers wave, wave + all waves, ...; the
// workgroup's waves meet in LDS and one non-returning atomic a workgroup adds
// them up (an atomic a container, all on the one total, serialised: 16384 of
// them took 80-200 us).
constexpr int CS_NT = 1024;

__global__ __launch_bounds__(CS_NT) void cv_card_sum(cr_gpu_roaring r, unsigned long long* total)
{
    __shared__ unsigned long long part[CS_NT / 64];
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t lane = __lane_id();
    const uint32_t nw = gridDim.x * (CS_NT / 64);
    unsigned long long n = 0;
    for (uint32_t c = blockIdx.x * (CS_NT / 64) + wave; c < r.n_containers; c += nw) n += container_count(r, c, lane);
    if (lane == 0) part[wave] = n;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long s = 0;
#pragma unroll
        for (int i = 0; i < CS_NT / 64; ++i) s += part[i];
        if (s) atomicAdd(total, s);
    }
}

__global__ void cv_zero_u64(unsigned long long* p) { *p = 0; }

// starts = exclusive scan of counts.  One workgroup per tile of 1024 counts:
// it sums every count before its tile (coalesced, eight loads per thread in
// flight) and scans its own tile, so no workgroup waits for another.
constexpr int SC_NT = 1024;

__device__ __forceinline__ unsigned long long block_sum64(unsigned long long v, unsigned long long* part)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    if (__lane_id() == 0) part[threadIdx.x >> 6] = v;
    __syncthreads();
    unsigned long long t = 0;
#pragma unroll
    for (int i = 0; i < SC_NT / 64; ++i) t += part[i];
    __syncthreads();
    return t;
}

__global__ __launch_bounds__(SC_NT) void cv_scan_u64(const uint64_t* __restrict__ counts, uint32_t n,
                                                     uint64_t* __restrict__ starts)
{
    __shared__ unsigned long long part[SC_NT / 64];
    const uint32_t t = threadIdx.x;
    const uint32_t tile0 = blockIdx.x * SC_NT;
    unsigned long long s = 0;
    for (uint32_t i0 = 0; i0 < tile0; i0 += 8 * SC_NT) {
        unsigned long long v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t i = i0 + j * SC_NT + t;
            v[j] = i < tile0 ? counts[i] : 0ull;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) s += v[j];
    }
    const unsigned long long base = block_sum64(s, part);
    const uint32_t i = tile0 + t;
    const unsigned long long x = i < n ? counts[i] : 0ull;
    unsigned long long incl = x;
    const uint32_t lane = __lane_id();
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned long long v = __shfl_up(incl, o, 64);
        if (lane >= static_cast<uint32_t>(o)) incl += v;
    }
    const uint32_t w = t >> 6;
    if (lane == 63) part[w] = incl;
    __syncthreads();
    unsigned long long pre = base + incl - x;
    for (uint32_t k = 0; k < w; ++k) pre += part[k];
    if (i < n) starts[i] = pre;
}

// A container of at most EW_STAGE ids is staged whole: one scan of the four
// chunks' counts (packed as 16-bit fields of a u64), the ids in order as u16
// in LDS, then one pass of coalesced int64 stores.  Denser containers go
// chunk by chunk.  LEAN: the input holds no run container, so no run image.
constexpr uint32_t EW_STAGE = 512u * 32u;  // 16384 ids

__device__ __forceinline__ unsigned long long block_excl_scan_u64(unsigned long long v, unsigned long long* part,
                                                                  unsigned long long& total)
{
    unsigned long long incl = v;
    const uint32_t lane = __lane_id();
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned long long x = __shfl_up(incl, o, 64);
        if (lane >= static_cast<uint32_t>(o)) incl += x;
    }
    const uint32_t w = threadIdx.x >> 6;
    if (lane == 63) part[w] = incl;
    __syncthreads();
    unsigned long long base = 0, t = 0;
#pragma unroll
    for (int i = 0; i < CV_NT / 64; ++i) {
        const unsigned long long x = part[i];
        base += (static_cast<uint32_t>(i) < w) ? x : 0ull;
        t += x;
    }
    __syncthreads();
    total = t;
    return base + incl - v;
}

template <bool LEAN>
__global__ __launch_bounds__(CV_NT) void cv_enum_write(cr_gpu_roaring r, const uint64_t* starts, uint64_t cap,
                                                       int64_t* __restrict__ out)
{
    struct NoImage {
        uint32_t w[1];
    };
    __shared__ std::conditional_t<LEAN, NoImage, Image> img;
    __shared__ uint16_t stage[EW_STAGE];
    __shared__ unsigned long long red64[CV_NT / 64];
    const uint32_t c = blockIdx.x;
    const uint32_t t = threadIdx.x;
    const uint8_t type = r.types[c];
    const uint32_t off = r.offsets[c];
    const int64_t base = static_cast<int64_t>(r.keys[c]) << 16;
    const uint64_t start = starts[c];
    if (type == CR_ARRAY) {
        const uint16_t* arr = r.array_data + off / 2u;
        const uint32_t card = r.cardinalities[c];
        for (uint32_t i0 = t; i0 < card; i0 += 4u * CV_NT) {  // four values a thread in flight
            uint32_t x[4];
#pragma unroll
            for (uint32_t k = 0; k < 4u; ++k) x[k] = i0 + CV_NT * k < card ? static_cast<uint32_t>(arr[i0 + CV_NT * k]) : 0u;
#pragma unroll
            for (uint32_t k = 0; k < 4u; ++k) {
                const uint32_t i = i0 + CV_NT * k;
                if (i < card && start + i < cap) st_stream(out + start + i, base | x[k]);
            }
        }
        return;
    }
    const uint32_t* words;
    if (type == CR_BITMAP) {
        words = reinterpret_cast<const uint32_t*>(r.bitmap_data + off / 8u);
    } else if (!LEAN && type == CR_RUN) {
        if constexpr (!LEAN) {
            expand_to_lds(CR_RUN, r.run_data + off / 2u, r.cardinalities[c], &img);
            words = img.w;
        }
    } else {
        return;
    }
    // thread t owns words 2t, 2t+1 of each 512-word chunk
    uint2 v[4];
#pragma unroll
    for (int ch = 0; ch < 4; ++ch) v[ch] = reinterpret_cast<const uint2*>(words)[ch * CV_NT + t];
    unsigned long long packed = 0;
#pragma unroll
    for (int ch = 0; ch < 4; ++ch)
        packed |= static_cast<unsigned long long>(__popc(v[ch].x) + __popc(v[ch].y)) << (16 * ch);
    unsigned long long totals;
    const unsigned long long pre = block_excl_scan_u64(packed, red64, totals);
    uint32_t tot[4], cbase[4];
    uint32_t all = 0;
#pragma unroll
    for (int ch = 0; ch < 4; ++ch) {
        tot[ch] = static_cast<uint32_t>(totals >> (16 * ch)) & 0xFFFFu;
        cbase[ch] = all;
        all += tot[ch];
    }
    if (all <= EW_STAGE) {
#pragma unroll
        for (int ch = 0; ch < 4; ++ch) {
            const uint32_t wi = ch * 512u + 2u * t;
            uint32_t pos = cbase[ch] + (static_cast<uint32_t>(pre >> (16 * ch)) & 0xFFFFu);
            for (uint32_t x = v[ch].x; x; x &= x - 1) stage[pos++] = static_cast<uint16_t>(32u * wi + __builtin_ctz(x));
            for (uint32_t x = v[ch].y; x; x &= x - 1)
                stage[pos++] = static_cast<uint16_t>(32u * (wi + 1u) + __builtin_ctz(x));
        }
        __syncthreads();
        for (uint32_t i = t; i < all; i += CV_NT)
            if (start + i < cap) st_stream(out + start + i, base | stage[i]);
        return;
    }
    uint64_t written = start;
#pragma unroll
    for (int ch = 0; ch < 4; ++ch) {
        const uint32_t wi = ch * 512u + 2u * t;
        uint32_t pos = static_cast<uint32_t>(pre >> (16 * ch)) & 0xFFFFu;
        for (uint32_t x = v[ch].x; x; x &= x - 1) stage[pos++] = static_cast<uint16_t>(32u * wi + __builtin_ctz(x));
        for (uint32_t x = v[ch].y; x; x &= x - 1)
            stage[pos++] = static_cast<uint16_t>(32u * (wi + 1u) + __builtin_ctz(x));
        __syncthreads();
        for (uint32_t i = t; i < tot[ch]; i += CV_NT)
            if (written + i < cap) st_stream(out + written + i, base | stage[i]);
        written += tot[ch];
        __syncthreads();
    }
}

// Arrays-only input: one wave per container, no LDS.
__global__ __launch_bounds__(CV_NT) void cv_enum_write_arrays(cr_gpu_roaring r, const uint64_t* starts, uint64_t cap,
                                                              int64_t* __restrict__ out)
{
    const uint32_t c = (blockIdx.x * CV_NT + threadIdx.x) >> 6;
    const uint32_t lane = __lane_id();
    if (c >= r.n_containers || r.types[c] != CR_ARRAY) return;
    const uint16_t* arr = r.array_data + r.offsets[c] / 2u;
    const uint32_t card = r.cardinalities[c];
    const int64_t base = static_cast<int64_t>(r.keys[c]) << 16;
    const uint64_t start = starts[c];
    for (uint32_t i0 = lane; i0 < card; i0 += 8u * 64u) {  // eight values a lane in flight
        uint32_t x[8];
#pragma unroll
        for (uint32_t k = 0; k < 8u; ++k) x[k] = i0 + 64u * k < card ? static_cast<uint32_t>(arr[i0 + 64u * k]) : 0u;
#pragma unroll
        for (uint32_t k = 0; k < 8u; ++k) {
            const uint32_t i = i0 + 64u * k;
            if (i < card && start + i < cap) st_stream(out + start + i, base | x[k]);
        }
    }
}

// ---- promote_to_bitmap ------------------------------------------------------
// One workgroup per container: keys and cards copied (a RUN card keeps its
// n_runs), type BITMAP at offset c * 8192, the 8 KiB image (copied, or built
// in LDS from an array / run container), and its key_index slot.  With no
// array or run container the bitmap pool is copied as it lies, container c
// taking pool words [c * 1024, c * 1024 + 1024) (src/promote.cu:268-276).
template <int NT, bool LEAN>
__global__ __launch_bounds__(NT) void cv_promote(cr_gpu_roaring src, bool all_bitmap, cr_gpu_roaring dst)
{
    constexpr int WPT = 2048 / NT;
    __shared__ alignas(16) uint32_t w[2048];
    __shared__ int32_t cover[LEAN ? 1 : 2048];
    const uint32_t c = blockIdx.x;
    const uint32_t t = threadIdx.x;
    const uint8_t type = src.types[c];
    uint4* o4 = reinterpret_cast<uint4*>(dst.bitmap_data + static_cast<uint64_t>(c) * 1024u);
    const uint32_t* words;
    const bool glob = all_bitmap || type == CR_BITMAP;
    if (glob) {
        words = reinterpret_cast<const uint32_t*>(all_bitmap ? src.bitmap_data + static_cast<uint64_t>(c) * 1024u
                                                             : src.bitmap_data + src.offsets[c] / 8u);
    } else if (type == CR_ARRAY || type == CR_RUN) {
        expand_img<NT>(type, (type == CR_ARRAY ? src.array_data : src.run_data) + src.offsets[c] / 2u,
                       src.cardinalities[c], w, LEAN ? nullptr : cover);
        words = w;
    } else {
#pragma unroll
        for (int j = 0; j < WPT; ++j) w[j * NT + t] = 0;
        __syncthreads();
        words = w;
    }
    if ((reinterpret_cast<uintptr_t>(words) & 15u) == 0) {
        constexpr int V = 512 / NT;
        uint4 v[V];
        if (glob) {
            const uint4* s4 = reinterpret_cast<const uint4*>(words);
#pragma unroll
            for (int j = 0; j < V; ++j) v[j] = ld_stream(s4 + j * NT + t);
        } else {
            const uint4* l4 = reinterpret_cast<const uint4*>(w);
#pragma unroll
            for (int j = 0; j < V; ++j) v[j] = l4[j * NT + t];
        }
#pragma unroll
        for (int j = 0; j < V; ++j) st_stream(o4 + j * NT + t, v[j]);
    } else {
        uint32_t* o = reinterpret_cast<uint32_t*>(o4);
        for (uint32_t i = t; i < 2048u; i += NT) o[i] = words[i];
    }
    if (t == 0) {
        const uint16_t key = src.keys[c];
        dst.keys[c] = key;
        dst.cardinalities[c] = src.cardinalities[c];
        dst.types[c] = CR_BITMAP;
        dst.offsets[c] = c * 8192u;
        if (dst.key_index && key <= dst.max_key) dst.key_index[key] = static_cast<uint16_t>(c);
    }
}

int deep_copy_impl(const cr_gpu_roaring* bm, hipStream_t s, cr_gpu_roaring* out)
{
    cr_gpu_roaring r{};
    r.n_containers = bm->n_containers;
    r.n_bitmap_containers = bm->n_bitmap_containers;
    r.n_array_containers = bm->n_array_containers;
    r.n_run_containers = bm->n_run_containers;
    r.universe_size = bm->universe_size;
    r.total_cardinality = bm->total_cardinality;
    r.negated = bm->negated;
    r.max_key = bm->max_key;
    r.array_pool_bytes = bm->array_pool_bytes;
    r.run_pool_bytes = bm->run_pool_bytes;
    const uint64_t n = bm->n_containers;
    if (n == 0) {  // src/promote.cu:194
        *out = r;
        return CR_OK;
    }
    // src/promote.cu:208-231: the bitmap pool copies n_bitmap x 8 KiB, the
    // array / run pools their byte counts, key_index max_key + 1 entries when
    // present and the universe is non-zero.
    const uint64_t bmp_words = (bm->bitmap_data && bm->n_bitmap_containers) ? bm->n_bitmap_containers * 1024ull : 0;
    const uint64_t arr_bytes = (bm->array_data && bm->array_pool_bytes) ? bm->array_pool_bytes : 0;
    const uint64_t run_bytes = (bm->run_data && bm->run_pool_bytes) ? bm->run_pool_bytes : 0;
    const uint64_t kidx_len = (bm->key_index && bm->universe_size > 0) ? bm->max_key + 1ull : 0;
    const OutLayout L = plan_out(n, kidx_len, bmp_words, (arr_bytes + 1) / 2, (run_bytes + 1) / 2);
    CR_RET(alloc_out(&r, L, n, kidx_len, bmp_words, (arr_bytes + 1) / 2, (run_bytes + 1) / 2, s));
    CopyList cl{};
    auto add = [&](const void* from, void* to, uint64_t bytes) {
        if (bytes) cl.seg[cl.n++] = {from, to, bytes};
    };
    add(bm->keys, r.keys, n * 2u);
    add(bm->types, r.types, n);
    add(bm->offsets, r.offsets, n * 4u);
    add(bm->cardinalities, r.cardinalities, n * 2u);
    add(bm->bitmap_data, r.bitmap_data, bmp_words * 8u);
    add(bm->array_data, r.array_data, arr_bytes);
    add(bm->run_data, r.run_data, run_bytes);
    add(bm->key_index, r.key_index, kidx_len * 2u);
    int rc;
    {
        CR_TIMED("cv_copy", s);
        rc = copy_segments(cl, s);
    }
    if (rc != CR_OK) {
        free_async(&r, s);
        return rc;
    }
    *out = r;
    return CR_OK;
}

int promote_impl(const cr_gpu_roaring* bm, hipStream_t s, cr_gpu_roaring* out)
{
    cr_gpu_roaring r{};
    const uint64_t n = bm->n_containers;
    if (n == 0) {  // GpuRoaring{} (src/promote.cu:236)
        *out = r;
        return CR_OK;
    }
    uint64_t kidx_len = 0;
    if (bm->universe_size > 0) {  // src/promote.cu:307-320
        r.max_key = std::min<uint32_t>((bm->universe_size - 1u) >> 16, 0xFFFFu);
        kidx_len = r.max_key + 1ull;
    }
    const OutLayout L = plan_out(n, kidx_len, n * 1024u, 0, 0);
    CR_RET(alloc_out(&r, L, n, kidx_len, n * 1024u, 0, 0, s));
    r.n_containers = static_cast<uint32_t>(n);
    r.n_bitmap_containers = static_cast<uint32_t>(n);
    r.universe_size = bm->universe_size;
    r.total_cardinality = bm->total_cardinality;
    r.negated = bm->negated;
    int rc = CR_OK;
    if (kidx_len) rc = fill_u16(r.key_index, 0xFFFFu, kidx_len, s);
    if (rc == CR_OK) {
        const bool all_bitmap = bm->n_array_containers == 0 && bm->n_run_containers == 0;
        CR_TIMED("cv_promote", s);
        if (bm->n_run_containers == 0)
            cv_promote<128, true><<<static_cast<uint32_t>(n), 128, 0, s>>>(*bm, all_bitmap, r);
        else
            cv_promote<CV_NT, false><<<static_cast<uint32_t>(n), CV_NT, 0, s>>>(*bm, all_bitmap, r);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) {
            set_error("cv_promote launch: %s", hipGetErrorString(e));
            rc = CR_ERR_HIP;
        }
    }
    if (rc != CR_OK) {
        free_async(&r, s);
        return rc;
    }
    *out = r;
    return CR_OK;
}

// The three launches of enumerate_ids over given counts/starts buffers
// (n_containers u64 each), untimed (enumerate_impl below times each launch).
// cv_enum_count writes every count and the scan every start, so neither
// buffer needs clearing first.
int enumerate_launch(const cr_gpu_roaring* bm, int64_t* d_out, uint64_t cap, uint64_t* counts, uint64_t* starts,
                     hipStream_t s)
{
    const uint32_t n = bm->n_containers;
    cv_enum_count<<<(n + 3) / 4, CV_NT, 0, s>>>(*bm, counts);
    CR_RET(scan_exclusive_u64(counts, n, starts, s));
    if (bm->n_bitmap_containers == 0 && bm->n_run_containers == 0)
        cv_enum_write_arrays<<<(n + 3) / 4, CV_NT, 0, s>>>(*bm, starts, cap, d_out);
    else if (bm->n_run_containers == 0)
        cv_enum_write<true><<<n, CV_NT, 0, s>>>(*bm, starts, cap, d_out);
    else
        cv_enum_write<false><<<n, CV_NT, 0, s>>>(*bm, starts, cap, d_out);
    CR_LAUNCH_CHECK();
    return CR_OK;
}

int enumerate_impl(const cr_gpu_roaring* bm, int64_t* d_out, uint64_t cap, hipStream_t s)
{
    if (bm->n_containers == 0 || bm->total_cardinality == 0) return CR_OK;  // src/to_csr.cu:163
    if (!d_out) {
        set_error("cr_enumerate_ids: null output");
        return CR_ERR_INVALID;
    }
    const uint32_t n = bm->n_containers;
    Scratch sc;
    CR_RET(sc.alloc(n * 16ull, s));
    uint64_t* counts = sc.at<uint64_t>(0);
    uint64_t* starts = sc.at<uint64_t>(n * 8ull);
    {
        CR_TIMED("cv_enum_count", s);
        cv_enum_count<<<(n + 3) / 4, CV_NT, 0, s>>>(*bm, counts);
    }
    {
        CR_TIMED("cv_enum_scan", s);
        CR_RET(scan_exclusive_u64(counts, n, starts, s));
    }
    {
        CR_TIMED("cv_enum_write", s);
        if (bm->n_bitmap_containers == 0 && bm->n_run_containers == 0)
            cv_enum_write_arrays<<<(n + 3) / 4, CV_NT, 0, s>>>(*bm, starts, cap, d_out);
        else if (bm->n_run_containers == 0)
            cv_enum_write<true><<<n, CV_NT, 0, s>>>(*bm, starts, cap, d_out);
        else
            cv_enum_write<false><<<n, CV_NT, 0, s>>>(*bm, starts, cap, d_out);
    }
    CR_LAUNCH_CHECK();
    return CR_OK;
}

// Ids that enumerate_ids writes for `bm`: the stored set, which for a negated
// bitmap is the complement of its logical set within [0, U).
uint64_t stored_cardinality(const cr_gpu_roaring* bm)
{
    if (!bm->negated) return bm->total_cardinality;
    return bm->universe_size > bm->total_cardinality ? bm->universe_size - bm->total_cardinality : 0;
}

}  // namespace

// ---- deep copy: up to eight byte ranges in one launch -----------------------
// One flat grid over the segments: segment i takes workgroups [blk0[i],
// blk0[i + 1]), one per 32 KiB (eight 16-byte loads in flight per thread), so
// small metadata segments cost a workgroup or two and the pool the rest.
constexpr uint64_t CV_COPY_BLK = 32768;

__global__ __launch_bounds__(256) void cv_copy(CopyList L)
{
    uint32_t s = 0;
    while (s + 1 < L.n && blockIdx.x >= L.blk0[s + 1]) ++s;
    const CopySeg g = L.seg[s];
    const uint64_t blk = blockIdx.x - L.blk0[s];
    const uint64_t lo = blk * CV_COPY_BLK, hi = std::min<uint64_t>(g.bytes, lo + CV_COPY_BLK);
    if (lo >= hi) return;
    const uint8_t* sb = static_cast<const uint8_t*>(g.src);
    uint8_t* db = static_cast<uint8_t*>(g.dst);
    uint64_t done = lo;
    if (((reinterpret_cast<uintptr_t>(g.src) | reinterpret_cast<uintptr_t>(g.dst)) & 15u) == 0) {
        const uint64_t n4 = (hi - lo) / 16u;
        const uint4* s4 = reinterpret_cast<const uint4*>(sb + lo);
        uint4* d4 = reinterpret_cast<uint4*>(db + lo);
        uint4 v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (threadIdx.x + k * 256u < n4) v[k] = ld_stream(s4 + threadIdx.x + k * 256u);
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (threadIdx.x + k * 256u < n4) st_stream(d4 + threadIdx.x + k * 256u, v[k]);
        done = lo + n4 * 16u;
    }
    for (uint64_t i = done + threadIdx.x; i < hi; i += 256u) db[i] = sb[i];
}

int copy_segments(const CopyList& L0, hipStream_t s)
{
    if (L0.n == 0) return CR_OK;
    CopyList L = L0;
    uint64_t total = 0;
    for (uint32_t i = 0; i < L.n; ++i) {
        L.blk0[i] = static_cast<uint32_t>(total);
        total += std::max<uint64_t>(1, (L.seg[i].bytes + CV_COPY_BLK - 1) / CV_COPY_BLK);
    }
    L.blk0[L.n] = static_cast<uint32_t>(total);
    if (total > 0xFFFFFFFFull) {
        set_error("copy_segments: %llu bytes exceed one grid", static_cast<unsigned long long>(total * CV_COPY_BLK));
        return CR_ERR_UNSUPPORTED;
    }
    cv_copy<<<static_cast<uint32_t>(total), 256, 0, s>>>(L);
    CR_LAUNCH_CHECK();
    return CR_OK;
}

int scan_exclusive_u64(const uint64_t* in, uint32_t n, uint64_t* out, hipStream_t s)
{
    if (n == 0) return CR_OK;
    cv_scan_u64<<<(n + SC_NT - 1) / SC_NT, SC_NT, 0, s>>>(in, n, out);
    CR_LAUNCH_CHECK();
    return CR_OK;
}

}  // namespace crimpl

using namespace crimpl;

extern "C" int cr_decompress_to_bitset(const cr_gpu_roaring* bm, uint32_t* d_out, uint32_t n_words,
                                       cr_stream_t stream)
{
    if (!bm || (n_words && !d_out)) {
        set_error("cr_decompress_to_bitset: invalid argument");
        return CR_ERR_INVALID;
    }
    if (n_words == 0) return CR_OK;
    hipStream_t s = as_stream(stream);
    const uint32_t regions = static_cast<uint32_t>((static_cast<uint64_t>(n_words) + 2047u) / 2048u);
    {
        CR_TIMED("cv_decompress", s);
        if (bm->n_run_containers == 0)
            cv_decompress<128, true><<<regions, 128, 0, s>>>(*bm, d_out, n_words);
        else
            cv_decompress<CV_NT, false><<<regions, CV_NT, 0, s>>>(*bm, d_out, n_words);
    }
    CR_LAUNCH_CHECK();
    return CR_OK;
}

extern "C" int cr_decompress_to_bitset_alloc(const cr_gpu_roaring* bm, cr_stream_t stream, uint32_t** d_out,
                                             uint32_t* n_words)
{
    if (!bm || !d_out || !n_words) {
        set_error("cr_decompress_to_bitset_alloc: invalid argument");
        return CR_ERR_INVALID;
    }
    *d_out = nullptr;
    *n_words = static_cast<uint32_t>((static_cast<uint64_t>(bm->universe_size) + 31u) / 32u);
    if (*n_words == 0) return CR_OK;  // src/decompress.cu:155-156
    CR_HIP_RET(hipMalloc(reinterpret_cast<void**>(d_out), *n_words * 4ull));
    const int rc = cr_decompress_to_bitset(bm, *d_out, *n_words, stream);
    if (rc != CR_OK) {
        (void)hipFree(*d_out);
        *d_out = nullptr;
    }
    return rc;
}

extern "C" int cr_enumerate_ids(const cr_gpu_roaring* bm, int64_t* d_out, uint64_t out_capacity, cr_stream_t stream)
{
    if (!bm) {
        set_error("cr_enumerate_ids: invalid argument");
        return CR_ERR_INVALID;
    }
    return enumerate_impl(bm, d_out, out_capacity, as_stream(stream));
}

// ---- cardinality ---------------------------------------------------------------
extern "C" int cr_cardinality(const cr_gpu_roaring* bm, cr_stream_t stream, uint64_t* out)
{
    if (!bm || !out) {
        set_error("cr_cardinality: invalid argument");
        return CR_ERR_INVALID;
    }
    uint64_t stored = 0;
    if (bm->n_containers) {
        hipStream_t s = as_stream(stream);
        Scratch sc;
        CR_RET(sc.alloc(256, s));
        unsigned long long* d_total = sc.at<unsigned long long>(0);
        {
            CR_TIMED("cv_card_sum", s);
            cv_zero_u64<<<1, 1, 0, s>>>(d_total);
            const uint32_t grid = std::min<uint32_t>((bm->n_containers + CS_NT / 64 - 1) / (CS_NT / 64), 2 * num_cus());
            cv_card_sum<<<grid, CS_NT, 0, s>>>(*bm, d_total);
        }
        CR_LAUNCH_CHECK();
        CR_RET(read_back(&stored, d_total, sizeof(stored), s));
    }
    // the logical set: a negated bitmap stores its complement within [0, U)
    *out = bm->negated ? (bm->universe_size > stored ? bm->universe_size - stored : 0) : stored;
    return CR_OK;
}

// ---- enumerate_ids without allocation ---------------------------------------
// For callers that cannot allocate device memory (code under graph capture,
// serving loops): the per-container counts and starts live in `scratch`, a
// file-scope device array sized for the most containers a bitmap can hold
// (65536 keys): 2 x 65536 u64 = 1 MiB, held by every device the library runs
// on until the process ends.  Host code never passes `scratch` itself to a
// kernel (in host code the name is a stand-in, not a device address): the
// entry point's first call on a device looks up that device's copy with
// hipGetSymbolAddress and keeps the address.  All calls on one device share
// the array, so calls that overlap on one device (different streams, or
// threads) race; calls on one stream are ordered.
constexpr uint32_t NOALLOC_MAX_CONTAINERS = 65536;
static __device__ __align__(256) uint64_t scratch[2 * NOALLOC_MAX_CONTAINERS];

namespace {
constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
uint64_t* g_scratch_ptr[NOALLOC_MAX_DEVICES] = {};

// The current device's copy of `scratch`, looked up once per device.
int scratch_of_current_device(uint64_t** out)
{
    int dev = -1;
    CR_HIP_RET(hipGetDevice(&dev));
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) {
        set_error("cr_enumerate_ids_noalloc: device %d outside the %d devices supported", dev, NOALLOC_MAX_DEVICES);
        return CR_ERR_UNSUPPORTED;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            set_error("cr_enumerate_ids_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                      hipGetErrorString(e));
            return CR_ERR_HIP;
        }
        g_scratch_ptr[dev] = static_cast<uint64_t*>(p);
    }
    *out = g_scratch_ptr[dev];
    return CR_OK;
}
}  // namespace

extern "C" int cr_enumerate_ids_noalloc(const cr_gpu_roaring* bm, int64_t* d_out, uint64_t out_capacity,
                                        cr_stream_t stream)
{
    if (!bm) {
        set_error("cr_enumerate_ids_noalloc: invalid argument");
        return CR_ERR_INVALID;
    }
    if (bm->n_containers == 0 || bm->total_cardinality == 0) return CR_OK;  // src/to_csr.cu:163
    if (!d_out) {
        set_error("cr_enumerate_ids_noalloc: null output");
        return CR_ERR_INVALID;
    }
    if (bm->n_containers > NOALLOC_MAX_CONTAINERS) {
        set_error("cr_enumerate_ids_noalloc: %u containers exceed the scratch bound of %u", bm->n_containers,
                  NOALLOC_MAX_CONTAINERS);
        return CR_ERR_INVALID;
    }
    uint64_t* sp = nullptr;
    CR_RET(scratch_of_current_device(&sp));
    return enumerate_launch(bm, d_out, out_capacity, sp, sp + NOALLOC_MAX_CONTAINERS, as_stream(stream));
}

extern "C" int cr_enumerate_ids_alloc(const cr_gpu_roaring* bm, cr_stream_t stream, int64_t** d_out,
                                      uint64_t* n_out)
{
    if (!bm || !d_out) {
        set_error("cr_enumerate_ids_alloc: invalid argument");
        return CR_ERR_INVALID;
    }
    *d_out = nullptr;
    if (n_out) *n_out = 0;
    if (bm->total_cardinality == 0) return CR_OK;  // src/to_csr.cu:213
    const uint64_t n = stored_cardinality(bm);
    if (n == 0) return CR_OK;
    CR_HIP_RET(hipMalloc(reinterpret_cast<void**>(d_out), n * 8ull));
    const int rc = enumerate_impl(bm, *d_out, n, as_stream(stream));
    if (rc != CR_OK) {
        (void)hipFree(*d_out);
        *d_out = nullptr;
        return rc;
    }
    if (n_out) *n_out = n;
    return CR_OK;
}

extern "C" int cr_promote_to_bitmap(const cr_gpu_roaring* bm, cr_stream_t stream, cr_gpu_roaring* out)
{
    if (!bm || !out) {
        set_error("cr_promote_to_bitmap: invalid argument");
        return CR_ERR_INVALID;
    }
    reset(out);
    return produced(promote_impl(bm, as_stream(stream), out), out, as_stream(stream));
}

extern "C" int cr_deep_copy(const cr_gpu_roaring* bm, cr_stream_t stream, cr_gpu_roaring* out)
{
    if (!bm || !out) {
        set_error("cr_deep_copy: invalid argument");
        return CR_ERR_INVALID;
    }
    reset(out);
    return produced(deep_copy_impl(bm, as_stream(stream), out), out, as_stream(stream));
}

extern "C" int cr_promote_auto(const cr_gpu_roaring* bm, cr_stream_t stream, int device_id, cr_gpu_roaring* out)
{
    if (!bm || !out) {
        set_error("cr_promote_auto: invalid argument");
        return CR_ERR_INVALID;
    }
    uint32_t thr = 0;
    CR_RET(cr_resolve_auto_threshold(bm->universe_size, device_id, &thr));
    reset(out);
    if (thr == CR_PROMOTE_ALL && (bm->n_array_containers > 0 || bm->n_run_containers > 0))
        return produced(promote_impl(bm, as_stream(stream), out), out, as_stream(stream));  // src/promote.cu:369-385
    return produced(deep_copy_impl(bm, as_stream(stream), out), out, as_stream(stream));
}

// The batch API (the reference's v2, v2/include/cu_roaring_v2/api.hpp): N
// Roaring bitmaps in one device block, CSR-style, with promote, multi_and,
// decompress and membership queries over the batch.
//
// Layout of the device block (our order; 256-byte aligned sections): the
// bitmap pool first, so every 8 KiB container is 8 KiB aligned in the block,
// then container_starts, key_index_starts, keys, types, offsets,
// cardinalities, key_indices, the array pool and the run pool.  Offsets are
// byte offsets into the pools, packed in global container order (the
// reference's rule, v2/src/upload.cpp:183-241), so they match the reference's.
// The host mirrors live in one malloc'd block.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "cu_roaring_v2/query.hpp"
#include "image.hpp"
#include "internal.hpp"

namespace crimpl {

namespace {

using cu_roaring::v2::GpuRoaringBatch;
using cu_roaring::v2::GpuRoaringView;

struct BatchLayout {
    size_t bmp = 0, cstart = 0, kstart = 0, keys = 0, types = 0, offs = 0, cards = 0, kidx = 0, arr = 0, run = 0;
    size_t total = 0;
};

BatchLayout plan_batch(uint64_t n, uint64_t T, uint64_t kidx, uint64_t bmp_words, uint64_t arr_u16, uint64_t run_u16)
{
    Carver c;
    BatchLayout L;
    L.bmp = c.add(bmp_words * 8);
    L.cstart = c.add((n + 1) * 4);
    L.kstart = c.add((n + 1) * 4);
    L.keys = c.add(T * 2);
    L.types = c.add(T);
    L.offs = c.add(T * 4);
    L.cards = c.add(T * 2);
    L.kidx = c.add(kidx * 2);
    L.arr = c.add(arr_u16 * 2);
    L.run = c.add(run_u16 * 2);
    L.total = c.total;
    return L;
}

void point_device(cr_roaring_batch* B, char* d, const BatchLayout& L, uint64_t T, uint64_t bmp_words,
                  uint64_t arr_u16, uint64_t run_u16)
{
    B->_alloc_base = d;
    B->container_starts = reinterpret_cast<uint32_t*>(d + L.cstart);
    B->key_index_starts = reinterpret_cast<uint32_t*>(d + L.kstart);
    B->keys = T ? reinterpret_cast<uint16_t*>(d + L.keys) : nullptr;
    B->types = T ? reinterpret_cast<uint8_t*>(d + L.types) : nullptr;
    B->offsets = T ? reinterpret_cast<uint32_t*>(d + L.offs) : nullptr;
    B->cardinalities = T ? reinterpret_cast<uint16_t*>(d + L.cards) : nullptr;
    B->key_indices = reinterpret_cast<uint16_t*>(d + L.kidx);
    B->bitmap_data = bmp_words ? reinterpret_cast<uint64_t*>(d + L.bmp) : nullptr;
    B->array_data = arr_u16 ? reinterpret_cast<uint16_t*>(d + L.arr) : nullptr;
    B->run_data = run_u16 ? reinterpret_cast<uint16_t*>(d + L.run) : nullptr;
}

// Host mirrors: total cardinality (u64), universe, container starts, key
// index starts, bitset counts (u32), one malloc.
struct HostMeta {
    uint64_t* card;
    uint32_t *universe, *cstart, *kstart, *nbm;
};

int alloc_host_meta(cr_roaring_batch* B, uint32_t n, HostMeta& m)
{
    const size_t bytes = n * 8ull + n * 4ull + 2 * (n + 1ull) * 4ull + n * 4ull;
    char* h = static_cast<char*>(std::calloc(1, bytes ? bytes : 8));
    if (!h) {
        set_error("host metadata allocation of %zu bytes failed", bytes);
        return CR_ERR_ALLOC;
    }
    m.card = reinterpret_cast<uint64_t*>(h);
    m.universe = reinterpret_cast<uint32_t*>(h + n * 8ull);
    m.cstart = m.universe + n;
    m.kstart = m.cstart + (n + 1);
    m.nbm = m.kstart + (n + 1);
    B->_host_meta_base = h;
    B->host_total_cardinalities = m.card;
    B->host_universe_sizes = m.universe;
    B->host_container_starts = m.cstart;
    B->host_key_index_starts = m.kstart;
    B->host_n_bitmap_containers = m.nbm;
    return CR_OK;
}

void release(cr_roaring_batch* B, hipStream_t s)
{
    if (B->_alloc_base) dev_free(B->_alloc_base, s);
    std::free(B->_host_meta_base);
    std::memset(B, 0, sizeof(*B));
}

PinnedStage g_batch_stage;

// ---- promote ------------------------------------------------------------------
// One workgroup per global container: its 8 KiB image (copied, or built in
// LDS from an array / run container) written to slot c, its popcount as the
// cardinality (65536 stored as 0), type BITMAP, offset c * 8192
// (v2/src/promote.cu:66-169).
// LEAN: one wavefront per container and no run difference array (batches
// without run containers), so more containers are in flight per CU.
template <int NT, bool LEAN>
__global__ __launch_bounds__(NT) void bt_promote(cr_roaring_batch src, uint32_t T, uint8_t* __restrict__ types,
                                                 uint32_t* __restrict__ offs, uint16_t* __restrict__ cards,
                                                 uint64_t* __restrict__ pool)
{
    constexpr int V = 512 / NT;  // 16-byte words per thread
    __shared__ alignas(16) uint32_t w[2048];
    __shared__ int32_t cover[LEAN ? 1 : 2048];
    __shared__ uint32_t red[NT / 64];
    const uint32_t c = blockIdx.x;
    const uint32_t t = threadIdx.x;
    const uint8_t type = src.types[c];
    const uint32_t off = src.offsets[c];
    uint4 v[V];
    if (type == CR_BITMAP) {
        const uint4* s4 = reinterpret_cast<const uint4*>(src.bitmap_data + off / 8u);
#pragma unroll
        for (int j = 0; j < V; ++j) v[j] = ld_stream(s4 + j * NT + t);
    } else {
        expand_img<NT>(type, (type == CR_ARRAY ? src.array_data : src.run_data) + off / 2u, src.cardinalities[c], w,
                       LEAN ? nullptr : cover);
        const uint4* s4 = reinterpret_cast<const uint4*>(w);
#pragma unroll
        for (int j = 0; j < V; ++j) v[j] = s4[j * NT + t];
    }
    uint4* d4 = reinterpret_cast<uint4*>(pool + static_cast<uint64_t>(c) * 1024u);
    uint32_t pc = 0;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        st_stream(d4 + j * NT + t, v[j]);
        pc += __popc(v[j].x) + __popc(v[j].y) + __popc(v[j].z) + __popc(v[j].w);
    }
    pc = block_sum<NT>(pc, red);
    if (t == 0) {
        types[c] = CR_BITMAP;
        offs[c] = c * 8192u;
        cards[c] = static_cast<uint16_t>(pc > 65535u ? 0u : pc);
    }
}

// ---- multi_and ------------------------------------------------------------------
// flags[i] = 1 iff anchor container i's key is present in every other input
// (v2/src/multi_and.cu:56-94).
__global__ __launch_bounds__(256) void bt_flags(cr_roaring_batch B, const uint32_t* __restrict__ idx, uint32_t n_in,
                                                uint32_t anchor_b, uint32_t a0, uint32_t an, uint64_t* flags)
{
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= an) return;
    const uint32_t key = B.keys[a0 + i];
    uint64_t ok = 1;
    for (uint32_t j = 0; j < n_in && ok; ++j) {
        const uint32_t b = idx[j];
        if (b == anchor_b) continue;
        const uint32_t k0 = B.key_index_starts[b], k1 = B.key_index_starts[b + 1];
        if (key >= k1 - k0 || B.key_indices[k0 + key] == 0xFFFFu) ok = 0;
    }
    flags[i] = ok;
}

__global__ void bt_starts(const uint64_t* flags, const uint64_t* pos, uint32_t an, uint32_t klen, uint32_t* cstart,
                          uint32_t* kstart, uint32_t* n_common)
{
    if (threadIdx.x != 0) return;
    const uint32_t m = static_cast<uint32_t>(pos[an - 1] + flags[an - 1]);
    cstart[0] = 0;
    cstart[1] = m;
    kstart[0] = 0;
    kstart[1] = klen;
    *n_common = m;
}

struct AndOut {
    uint16_t* keys;
    uint8_t* types;
    uint32_t* offs;
    uint16_t* cards;
    uint16_t* kidx;
    uint64_t* pool;
    unsigned long long* total;
};

// One workgroup per anchor container that survived: the inputs' container
// addresses gathered into LDS, then the AND of the 1024 words with the loads
// of four inputs in flight per step; popcount into the cardinality and the
// batch total (v2/src/multi_and.cu:126-205).
constexpr uint32_t MA_MAX_INPUTS = 4096;

__global__ __launch_bounds__(CV_NT) void bt_and(cr_roaring_batch B, const uint32_t* __restrict__ idx, uint32_t n_in,
                                                uint32_t a0, const uint64_t* __restrict__ flags,
                                                const uint64_t* __restrict__ pos, AndOut o)
{
    __shared__ const uint4* src[MA_MAX_INPUTS];
    __shared__ uint32_t red[CV_NT / 64];
    const uint32_t i = blockIdx.x;
    const uint32_t t = threadIdx.x;
    if (flags[i] == 0) return;
    const uint32_t k = static_cast<uint32_t>(pos[i]);
    const uint32_t key = B.keys[a0 + i];
    for (uint32_t j = t; j < n_in; j += CV_NT) {
        const uint32_t b = idx[j];
        const uint32_t local = B.key_indices[B.key_index_starts[b] + key];
        const uint32_t gcid = B.container_starts[b] + local;
        src[j] = reinterpret_cast<const uint4*>(B.bitmap_data + B.offsets[gcid] / 8u);
    }
    __syncthreads();
    uint4 acc[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) acc[h] = make_uint4(~0u, ~0u, ~0u, ~0u);
    uint32_t j = 0;
    for (; j + 4 <= n_in; j += 4) {
        uint4 v[4][2];
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int h = 0; h < 2; ++h) v[q][h] = ld_stream(src[j + q] + h * CV_NT + t);
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                acc[h].x &= v[q][h].x;
                acc[h].y &= v[q][h].y;
                acc[h].z &= v[q][h].z;
                acc[h].w &= v[q][h].w;
            }
    }
    for (; j < n_in; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint4 v = ld_stream(src[j] + h * CV_NT + t);
            acc[h].x &= v.x;
            acc[h].y &= v.y;
            acc[h].z &= v.z;
            acc[h].w &= v.w;
        }
    uint4* d4 = reinterpret_cast<uint4*>(o.pool + static_cast<uint64_t>(k) * 1024u);
    uint32_t pc = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        st_stream(d4 + h * CV_NT + t, acc[h]);
        pc += __popc(acc[h].x) + __popc(acc[h].y) + __popc(acc[h].z) + __popc(acc[h].w);
    }
    pc = block_sum<CV_NT>(pc, red);
    if (t == 0) {
        o.keys[k] = static_cast<uint16_t>(key);
        o.types[k] = CR_BITMAP;
        o.offs[k] = k * 8192u;
        o.cards[k] = static_cast<uint16_t>(pc > 65535u ? 0u : pc);
        o.kidx[key] = static_cast<uint16_t>(k);
        atomicAdd(o.total, static_cast<unsigned long long>(pc));
    }
}

// Up to 64 inputs: one wavefront per surviving anchor container (grid-stride),
// lane j resolves input j's container address, and the wave streams each
// input's 8 KiB as eight 16-byte loads per lane with the next input's loads
// issued before the current one is ANDed in.
__global__ __launch_bounds__(256) void bt_and_wave(cr_roaring_batch B, const uint32_t* __restrict__ idx, uint32_t n_in,
                                                   uint32_t a0, uint32_t an, const uint64_t* __restrict__ flags,
                                                   const uint64_t* __restrict__ pos, AndOut o)
{
    __shared__ unsigned long long wave_total[4];
    const uint32_t lane = __lane_id();
    const uint32_t n_waves = gridDim.x * 4u;
    unsigned long long my_total = 0;
    for (uint32_t i = (blockIdx.x * 256u + threadIdx.x) >> 6; i < an; i += n_waves) {
        if (flags[i] == 0) continue;  // the whole wavefront skips
        const uint32_t k = static_cast<uint32_t>(pos[i]);
        const uint32_t key = B.keys[a0 + i];
        unsigned long long my_p = 0;
        if (lane < n_in) {
            const uint32_t b = idx[lane];
            const uint32_t gcid = B.container_starts[b] + B.key_indices[B.key_index_starts[b] + key];
            my_p = reinterpret_cast<unsigned long long>(B.bitmap_data + B.offsets[gcid] / 8u);
        }
        auto load8 = [&](uint32_t j, uint4 (&x)[8]) {
            const uint4* p4 = reinterpret_cast<const uint4*>(__shfl(my_p, static_cast<int>(j), 64));
#pragma unroll
            for (int q = 0; q < 8; ++q) x[q] = ld_stream(p4 + lane + 64 * q);
        };
        uint4 acc[8], cur[8], nxt[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) acc[q] = make_uint4(~0u, ~0u, ~0u, ~0u);
        load8(0, cur);
        for (uint32_t j = 0; j < n_in; ++j) {
            if (j + 1 < n_in) load8(j + 1, nxt);
#pragma unroll
            for (int q = 0; q < 8; ++q)
                acc[q] = make_uint4(acc[q].x & cur[q].x, acc[q].y & cur[q].y, acc[q].z & cur[q].z, acc[q].w & cur[q].w);
#pragma unroll
            for (int q = 0; q < 8; ++q) cur[q] = nxt[q];
        }
        uint4* d4 = reinterpret_cast<uint4*>(o.pool + static_cast<uint64_t>(k) * 1024u);
        uint32_t pc = 0;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            st_stream(d4 + lane + 64 * q, acc[q]);
            pc += __popc(acc[q].x) + __popc(acc[q].y) + __popc(acc[q].z) + __popc(acc[q].w);
        }
        pc = wave_sum(pc);
        my_total += pc;
        if (lane == 0) {
            o.keys[k] = static_cast<uint16_t>(key);
            o.types[k] = CR_BITMAP;
            o.offs[k] = k * 8192u;
            o.cards[k] = static_cast<uint16_t>(pc > 65535u ? 0u : pc);
            o.kidx[key] = static_cast<uint16_t>(k);
        }
    }
    if (lane == 0) wave_total[threadIdx.x >> 6] = my_total;
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned long long s = wave_total[0] + wave_total[1] + wave_total[2] + wave_total[3];
        if (s) atomicAdd(o.total, s);
    }
}

// ---- decompress -----------------------------------------------------------------
// Owner of global container c: the b with container_starts[b] <= c <
// container_starts[b + 1], found with 64 probes per step by one wavefront.
__device__ uint32_t wave_owner(const uint32_t* starts, uint32_t n_bitmaps, uint32_t c)
{
    const uint32_t lane = __lane_id();
    uint32_t lo = 0, hi = n_bitmaps;  // answer in [lo, hi): last b with starts[b] <= c
    while (hi - lo > 1) {
        const uint32_t step = (hi - lo + 63) / 64;
        const uint32_t p = lo + lane * step;
        const bool le = p < hi && starts[p] <= c;
        const uint32_t cnt = static_cast<uint32_t>(__popcll(__ballot(le)));  // probes at or below c
        const uint32_t nlo = lo + (cnt - 1) * step;
        hi = min(hi, nlo + step);
        lo = nlo;
    }
    // several bitmaps may start at c (empty ones): take the last, which owns c
    return lo;
}

// One workgroup per global container: its 1024-word window of bitmap b's
// slot (clipped at the slot end) stored for a bitmap container, OR-ed into
// the buffer for an array / run container (v2/src/decompress.cu:42-145).
template <int NT, bool LEAN>
__global__ __launch_bounds__(NT) void bt_decompress(cr_roaring_batch B, uint64_t* __restrict__ out,
                                                    uint64_t words_each)
{
    __shared__ alignas(16) uint32_t w[2048];
    __shared__ int32_t cover[LEAN ? 1 : 2048];
    __shared__ uint32_t s_b;
    const uint32_t c = blockIdx.x;
    const uint32_t t = threadIdx.x;
    if (t < 64) {
        const uint32_t b = wave_owner(B.container_starts, B.n_bitmaps, c);
        if (t == 0) s_b = b;
    }
    __syncthreads();
    const uint32_t b = s_b;
    const uint64_t base = static_cast<uint64_t>(b) * words_each, end = base + words_each;
    const uint64_t wb = base + static_cast<uint64_t>(B.keys[c]) * 1024u;
    if (wb >= end) return;
    const uint32_t window = static_cast<uint32_t>(min<uint64_t>(1024u, end - wb));
    uint64_t* dst = out + wb;
    const uint8_t type = B.types[c];
    const uint32_t off = B.offsets[c];
    constexpr int V = 512 / NT;  // 16-byte vectors per thread for a whole window
    const bool vec = window == 1024u && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0;
    uint4* d4 = reinterpret_cast<uint4*>(dst);
    if (type == CR_BITMAP) {
        const uint64_t* src = B.bitmap_data + off / 8u;
        if (vec && (reinterpret_cast<uintptr_t>(src) & 15u) == 0) {
            const uint4* s4 = reinterpret_cast<const uint4*>(src);
            uint4 v[V];
#pragma unroll
            for (int j = 0; j < V; ++j) v[j] = ld_stream(s4 + j * NT + t);
#pragma unroll
            for (int j = 0; j < V; ++j) st_stream(d4 + j * NT + t, v[j]);
        } else {
            for (uint32_t i = t; i < window; i += NT) dst[i] = src[i];
        }
        return;
    }
    uint4 prior[V];
    if (vec) {  // the caller's words are read while the image is built
#pragma unroll
        for (int j = 0; j < V; ++j) prior[j] = ld_stream(d4 + j * NT + t);
    }
    expand_img<NT>(type, (type == CR_ARRAY ? B.array_data : B.run_data) + off / 2u, B.cardinalities[c], w,
                   LEAN ? nullptr : cover);
    if (vec) {
        const uint4* l4 = reinterpret_cast<const uint4*>(w);
#pragma unroll
        for (int j = 0; j < V; ++j) {
            const uint4 m = l4[j * NT + t];
            st_stream(d4 + j * NT + t,
                      make_uint4(prior[j].x | m.x, prior[j].y | m.y, prior[j].z | m.z, prior[j].w | m.w));
        }
    } else {
        const uint64_t* img64 = reinterpret_cast<const uint64_t*>(w);
        for (uint32_t i = t; i < window; i += NT) dst[i] |= img64[i];
    }
}

// ---- queries --------------------------------------------------------------------
__global__ __launch_bounds__(256) void bt_contains(GpuRoaringBatch B, const uint32_t* __restrict__ bidx, uint32_t b,
                                                   const uint32_t* __restrict__ ids, uint64_t n,
                                                   uint8_t* __restrict__ out)
{
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * 256u;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x; i < n; i += stride)
        out[i] = cu_roaring::v2::contains(B, bidx ? bidx[i] : b, ids[i]) ? 1 : 0;
}

__global__ __launch_bounds__(256) void bt_view_contains(GpuRoaringView v, const uint32_t* __restrict__ ids, uint64_t n,
                                                        uint8_t* __restrict__ out)
{
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * 256u;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x; i < n; i += stride)
        out[i] = cu_roaring::v2::contains(v, ids[i]) ? 1 : 0;
}

uint32_t query_grid(uint64_t n) { return static_cast<uint32_t>(std::max<uint64_t>(1, std::min<uint64_t>((n + 255) / 256, 1u << 20))); }

}  // namespace
}  // namespace crimpl

using namespace crimpl;

extern "C" int cr_upload_batch(const cr_host_container* const* bitmaps, const uint32_t* n_containers,
                               uint32_t n_bitmaps, cr_stream_t stream, cr_roaring_batch* out)
{
    if (!out || (n_bitmaps && (!bitmaps || !n_containers))) {
        set_error("cr_upload_batch: invalid argument");
        return CR_ERR_INVALID;
    }
    std::memset(out, 0, sizeof(*out));
    if (n_bitmaps == 0) return CR_OK;  // v2/src/upload.cpp:323
    uint64_t T = 0, bmp_words = 0, arr_u16 = 0, run_u16 = 0, kidx = 0, n_bmp = 0;
    for (uint32_t b = 0; b < n_bitmaps; ++b) {
        const uint32_t nc = n_containers[b];
        if (nc && !bitmaps[b]) {
            set_error("cr_upload_batch: bitmap %u is null", b);
            return CR_ERR_INVALID;
        }
        for (uint32_t i = 0; i < nc; ++i) {
            const cr_host_container& h = bitmaps[b][i];
            const bool bad_type = h.typecode != CR_TC_BITSET && h.typecode != CR_TC_ARRAY && h.typecode != CR_TC_RUN;
            if (bad_type || h.cardinality < 0 || (h.cardinality > 0 && !h.data) ||
                (i > 0 && bitmaps[b][i - 1].key >= h.key)) {
                set_error("cr_upload_batch: bitmap %u container %u is malformed (type, order or payload)", b, i);
                return CR_ERR_INVALID;
            }
            if (h.typecode == CR_TC_BITSET) {
                bmp_words += 1024;
                ++n_bmp;
            } else if (h.typecode == CR_TC_ARRAY) {
                arr_u16 += static_cast<uint64_t>(h.cardinality);
            } else {
                run_u16 += 2ull * static_cast<uint64_t>(h.cardinality);
            }
        }
        T += nc;
        if (nc) kidx += static_cast<uint64_t>(bitmaps[b][nc - 1].key) + 1u;
    }
    if (bmp_words * 8 > 0xFFFFFFFFull || arr_u16 * 2 > 0xFFFFFFFFull || run_u16 * 2 > 0xFFFFFFFFull ||
        T > 0xFFFFFFFFull) {
        set_error("cr_upload_batch: a pool exceeds the 32-bit byte offsets of the batch format");
        return CR_ERR_UNSUPPORTED;
    }
    hipStream_t s = as_stream(stream);
    const BatchLayout L = plan_batch(n_bitmaps, T, kidx, bmp_words, arr_u16, run_u16);
    HostMeta m{};
    CR_RET(alloc_host_meta(out, n_bitmaps, m));
    std::lock_guard<std::mutex> lock(g_batch_stage.mu);
    int rc = g_batch_stage.reserve(L.total);
    if (rc != CR_OK) {
        release(out, s);
        return rc;
    }
    char* h = static_cast<char*>(g_batch_stage.ptr);
    auto* cs = reinterpret_cast<uint32_t*>(h + L.cstart);
    auto* ks = reinterpret_cast<uint32_t*>(h + L.kstart);
    auto* keys = reinterpret_cast<uint16_t*>(h + L.keys);
    auto* types = reinterpret_cast<uint8_t*>(h + L.types);
    auto* offs = reinterpret_cast<uint32_t*>(h + L.offs);
    auto* cards = reinterpret_cast<uint16_t*>(h + L.cards);
    auto* ki = reinterpret_cast<uint16_t*>(h + L.kidx);
    auto* bmp = reinterpret_cast<uint64_t*>(h + L.bmp);
    auto* arr = reinterpret_cast<uint16_t*>(h + L.arr);
    auto* run = reinterpret_cast<uint16_t*>(h + L.run);
    std::memset(ki, 0xFF, kidx * 2);
    uint64_t gid = 0, bc = 0, ac = 0, rcur = 0, kc = 0;
    cs[0] = ks[0] = 0;
    for (uint32_t b = 0; b < n_bitmaps; ++b) {
        const uint32_t nc = n_containers[b];
        uint64_t card = 0;
        uint32_t nb = 0;
        for (uint32_t i = 0; i < nc; ++i, ++gid) {
            const cr_host_container& c = bitmaps[b][i];
            keys[gid] = c.key;
            ki[kc + c.key] = static_cast<uint16_t>(i);
            if (c.typecode == CR_TC_BITSET) {  // v2/src/upload.cpp:190-204
                types[gid] = CR_BITMAP;
                offs[gid] = static_cast<uint32_t>(bc * 8);
                cards[gid] = static_cast<uint16_t>(c.cardinality > 65535 ? 0 : c.cardinality);
                std::memcpy(bmp + bc, c.data, 8192);
                bc += 1024;
                card += static_cast<uint64_t>(c.cardinality);
                ++nb;
            } else if (c.typecode == CR_TC_ARRAY) {
                types[gid] = CR_ARRAY;
                offs[gid] = static_cast<uint32_t>(ac * 2);
                cards[gid] = static_cast<uint16_t>(c.cardinality);
                std::memcpy(arr + ac, c.data, static_cast<size_t>(c.cardinality) * 2u);
                ac += static_cast<uint64_t>(c.cardinality);
                card += static_cast<uint64_t>(c.cardinality);
            } else {
                types[gid] = CR_RUN;
                offs[gid] = static_cast<uint32_t>(rcur * 2);
                cards[gid] = static_cast<uint16_t>(c.cardinality);
                const uint16_t* r = static_cast<const uint16_t*>(c.data);
                std::memcpy(run + rcur, r, static_cast<size_t>(c.cardinality) * 4u);
                for (int32_t k = 0; k < c.cardinality; ++k) card += static_cast<uint64_t>(r[2 * k + 1]) + 1u;
                rcur += 2ull * static_cast<uint64_t>(c.cardinality);
            }
        }
        const uint32_t klen = nc ? static_cast<uint32_t>(bitmaps[b][nc - 1].key) + 1u : 0u;
        kc += klen;
        cs[b + 1] = static_cast<uint32_t>(gid);
        ks[b + 1] = static_cast<uint32_t>(kc);
        m.card[b] = card;
        m.universe[b] = nc ? (klen << 16) : 0u;  // (max_key + 1) << 16 in 32 bits
        m.nbm[b] = nb;
    }
    std::memcpy(m.cstart, cs, (n_bitmaps + 1ull) * 4);
    std::memcpy(m.kstart, ks, (n_bitmaps + 1ull) * 4);
    void* d = nullptr;
    rc = dev_alloc(&d, L.total, s);
    if (rc != CR_OK) {
        release(out, s);
        return rc;
    }
    point_device(out, static_cast<char*>(d), L, T, bmp_words, arr_u16, run_u16);
    out->n_bitmaps = n_bitmaps;
    out->total_containers = static_cast<uint32_t>(T);
    out->n_bitmap_containers_total = static_cast<uint32_t>(n_bmp);
    out->array_pool_bytes = static_cast<uint32_t>(arr_u16 * 2);
    out->run_pool_bytes = static_cast<uint32_t>(run_u16 * 2);
    hipError_t e = hipMemcpyAsync(d, h, L.total, hipMemcpyHostToDevice, s);
    rc = e == hipSuccess ? sync_stream(s) : CR_ERR_HIP;  // the staging buffer is reused by the next call
    if (e != hipSuccess) set_error("cr_upload_batch: %s", hipGetErrorString(e));
    if (rc != CR_OK) release(out, s);
    return rc;
}

extern "C" int cr_free_batch(cr_roaring_batch* batch)
{
    if (!batch) return CR_OK;
    if (batch->_alloc_base) CR_HIP_RET(hipDeviceSynchronize());  // free_batch frees synchronously
    release(batch, nullptr);
    return CR_OK;
}

extern "C" int cr_promote_batch(const cr_roaring_batch* in, cr_stream_t stream, cr_roaring_batch* out)
{
    if (!in || !out) {
        set_error("cr_promote_batch: invalid argument");
        return CR_ERR_INVALID;
    }
    std::memset(out, 0, sizeof(*out));
    const uint32_t n = in->n_bitmaps;
    if (n == 0) return CR_OK;  // v2/src/promote.cu:216
    const uint64_t T = in->total_containers;
    const uint64_t kidx = in->host_key_index_starts[n];
    hipStream_t s = as_stream(stream);
    HostMeta m{};
    CR_RET(alloc_host_meta(out, n, m));
    std::memcpy(m.card, in->host_total_cardinalities, n * 8ull);
    std::memcpy(m.universe, in->host_universe_sizes, n * 4ull);
    std::memcpy(m.cstart, in->host_container_starts, (n + 1ull) * 4);
    std::memcpy(m.kstart, in->host_key_index_starts, (n + 1ull) * 4);
    for (uint32_t b = 0; b < n; ++b) m.nbm[b] = m.cstart[b + 1] - m.cstart[b];
    const BatchLayout L = plan_batch(n, T, kidx, T * 1024, 0, 0);
    void* d = nullptr;
    int rc = dev_alloc(&d, L.total, s);
    if (rc != CR_OK) {
        release(out, s);
        return rc;
    }
    point_device(out, static_cast<char*>(d), L, T, T * 1024, 0, 0);
    out->n_bitmaps = n;
    out->total_containers = static_cast<uint32_t>(T);
    out->n_bitmap_containers_total = static_cast<uint32_t>(T);
    CopyList cl{};
    cl.seg[cl.n++] = {in->container_starts, out->container_starts, (n + 1ull) * 4};
    cl.seg[cl.n++] = {in->key_index_starts, out->key_index_starts, (n + 1ull) * 4};
    if (T) cl.seg[cl.n++] = {in->keys, out->keys, T * 2};
    if (kidx) cl.seg[cl.n++] = {in->key_indices, out->key_indices, kidx * 2};
    rc = copy_segments(cl, s);
    if (rc == CR_OK && T) {
        CR_TIMED("bt_promote", s);
        if (in->run_pool_bytes == 0)
            bt_promote<128, true><<<static_cast<uint32_t>(T), 128, 0, s>>>(*in, static_cast<uint32_t>(T), out->types,
                                                                          out->offsets, out->cardinalities,
                                                                          out->bitmap_data);
        else
            bt_promote<CV_NT, false><<<static_cast<uint32_t>(T), CV_NT, 0, s>>>(
                *in, static_cast<uint32_t>(T), out->types, out->offsets, out->cardinalities, out->bitmap_data);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) {
            set_error("bt_promote launch: %s", hipGetErrorString(e));
            rc = CR_ERR_HIP;
        }
    }
    if (rc != CR_OK) release(out, s);
    return rc;
}

extern "C" int cr_batch_make_view(const cr_roaring_batch* batch, uint32_t b, cr_batch_view* out)
{
    if (!batch || !out) {
        set_error("cr_batch_make_view: invalid argument");
        return CR_ERR_INVALID;
    }
    if (b >= batch->n_bitmaps) {
        set_error("make_view: bitmap_idx %u out of range for batch of size %u", b, batch->n_bitmaps);
        return CR_ERR_RANGE;
    }
    std::memset(out, 0, sizeof(*out));
    if (!batch->host_container_starts) return CR_OK;
    const uint32_t c0 = batch->host_container_starts[b], c1 = batch->host_container_starts[b + 1];
    const uint32_t k0 = batch->host_key_index_starts[b], k1 = batch->host_key_index_starts[b + 1];
    out->n_containers = c1 - c0;
    out->max_key = k1 > k0 ? k1 - k0 - 1u : 0u;  // v2/src/upload.cpp:393-395
    if (out->n_containers) {
        out->keys = batch->keys + c0;
        out->types = batch->types + c0;
        out->offsets = batch->offsets + c0;
        out->cardinalities = batch->cardinalities + c0;
        out->key_index = batch->key_indices + k0;
    }
    out->bitmap_data = batch->bitmap_data;
    out->array_data = batch->array_data;
    out->run_data = batch->run_data;
    return CR_OK;
}

namespace {
int empty_one_batch(hipStream_t s, cr_roaring_batch* out)
{
    // one empty bitmap: both CSR start arrays {0, 0} (v2/src/multi_and.cu:207-242)
    HostMeta m{};
    CR_RET(alloc_host_meta(out, 1, m));
    void* d = nullptr;
    int rc = dev_alloc(&d, 256, s);
    if (rc == CR_OK) rc = fill_u32(static_cast<uint32_t*>(d), 0u, 4, s);
    if (rc != CR_OK) {
        if (d) dev_free(d, s);
        release(out, s);
        return rc;
    }
    out->_alloc_base = d;
    out->container_starts = static_cast<uint32_t*>(d);
    out->key_index_starts = static_cast<uint32_t*>(d) + 2;
    out->n_bitmaps = 1;
    return CR_OK;
}
}  // namespace

extern "C" int cr_batch_multi_and(const cr_roaring_batch* batch, const uint32_t* host_indices, uint32_t n_inputs,
                                  cr_stream_t stream, cr_roaring_batch* out)
{
    if (!batch || !out) {
        set_error("cr_batch_multi_and: invalid argument");
        return CR_ERR_INVALID;
    }
    if (n_inputs == 0 || !host_indices) {
        set_error("multi_and: n_inputs must be >= 1 and input_indices non-null");
        return CR_ERR_INVALID;
    }
    const uint32_t* hs = batch->host_container_starts;
    for (uint32_t k = 0; k < n_inputs; ++k) {  // v2/src/multi_and.cu:244-274
        const uint32_t b = host_indices[k];
        if (b >= batch->n_bitmaps) {
            set_error("multi_and: input_indices[%u] = %u out of range for batch of size %u", k, b, batch->n_bitmaps);
            return CR_ERR_RANGE;
        }
        if (batch->host_n_bitmap_containers[b] != hs[b + 1] - hs[b]) {
            set_error("multi_and: input_indices[%u] = %u has non-bitmap containers; call promote_batch first", k, b);
            return CR_ERR_INVALID;
        }
    }
    if (n_inputs > MA_MAX_INPUTS) {
        set_error("multi_and: %u inputs exceed this build's limit of %u", n_inputs, MA_MAX_INPUTS);
        return CR_ERR_UNSUPPORTED;
    }
    std::memset(out, 0, sizeof(*out));
    hipStream_t s = as_stream(stream);
    uint32_t ap = 0;
    for (uint32_t k = 0; k < n_inputs; ++k) {
        const uint32_t b = host_indices[k];
        if (hs[b + 1] == hs[b]) return empty_one_batch(s, out);
        if (hs[b + 1] - hs[b] < hs[host_indices[ap] + 1] - hs[host_indices[ap]]) ap = k;
    }
    const uint32_t ab = host_indices[ap];
    const uint32_t a0 = hs[ab], an = hs[ab + 1] - hs[ab];
    const uint32_t klen = batch->host_key_index_starts[ab + 1] - batch->host_key_index_starts[ab];

    Carver sc_c;
    const size_t o_idx = sc_c.add(n_inputs * 4ull), o_flags = sc_c.add(an * 8ull), o_pos = sc_c.add(an * 8ull),
                 o_tot = sc_c.add(16);
    Scratch sc;
    CR_RET(sc.alloc(sc_c.total, s));
    uint32_t* d_idx = sc.at<uint32_t>(o_idx);
    uint64_t* flags = sc.at<uint64_t>(o_flags);
    uint64_t* pos = sc.at<uint64_t>(o_pos);
    auto* total = sc.at<unsigned long long>(o_tot);
    uint32_t* n_common_d = sc.at<uint32_t>(o_tot + 8);
    CR_HIP_RET(hipMemcpyAsync(d_idx, host_indices, n_inputs * 4ull, hipMemcpyHostToDevice, s));
    CR_RET(fill_u32(reinterpret_cast<uint32_t*>(total), 0u, 4, s));
    {
        CR_TIMED("bt_flags", s);
        bt_flags<<<(an + 255) / 256, 256, 0, s>>>(*batch, d_idx, n_inputs, ab, a0, an, flags);
    }
    CR_LAUNCH_CHECK();
    CR_RET(scan_exclusive_u64(flags, an, pos, s));

    // output sized for every anchor container (the count is known only on the device)
    const BatchLayout L = plan_batch(1, an, klen, an * 1024ull, 0, 0);
    HostMeta m{};
    CR_RET(alloc_host_meta(out, 1, m));
    void* d = nullptr;
    int rc = dev_alloc(&d, L.total, s);
    if (rc != CR_OK) {
        release(out, s);
        return rc;
    }
    point_device(out, static_cast<char*>(d), L, an, an * 1024ull, 0, 0);
    if (klen) rc = fill_u16(out->key_indices, 0xFFFFu, klen, s);
    uint32_t n_common = 0;
    unsigned long long tot = 0;
    if (rc == CR_OK) {
        bt_starts<<<1, 64, 0, s>>>(flags, pos, an, klen, out->container_starts, out->key_index_starts, n_common_d);
        AndOut o{out->keys, out->types, out->offsets, out->cardinalities, out->key_indices, out->bitmap_data, total};
        {
            CR_TIMED("bt_and", s);
            if (n_inputs <= 64) {
                const uint32_t grid = std::min<uint32_t>((an + 3) / 4, 4u * num_cus());
                bt_and_wave<<<grid, 256, 0, s>>>(*batch, d_idx, n_inputs, a0, an, flags, pos, o);
            } else {
                bt_and<<<an, CV_NT, 0, s>>>(*batch, d_idx, n_inputs, a0, flags, pos, o);
            }
        }
        HostSlotGuard hs;  // both totals come back through one pinned slot
        rc = hs.acquire();
        if (rc == CR_OK) {
            char* hp = static_cast<char*>(hs.slot.host);
            hipError_t e = hipGetLastError();
            if (e == hipSuccess) e = hipMemcpyAsync(hp, total, 8, hipMemcpyDeviceToHost, s);
            if (e == hipSuccess) e = hipMemcpyAsync(hp + 8, n_common_d, 4, hipMemcpyDeviceToHost, s);
            if (e != hipSuccess) {
                set_error("cr_batch_multi_and: %s", hipGetErrorString(e));
                rc = CR_ERR_HIP;
            } else {
                rc = sync_stream(s);
            }
            if (rc == CR_OK) {
                std::memcpy(&tot, hp, 8);
                std::memcpy(&n_common, hp + 8, 4);
            }
        }
    }
    if (rc != CR_OK) {
        release(out, s);
        return rc;
    }
    out->n_bitmaps = 1;
    out->total_containers = n_common;
    out->n_bitmap_containers_total = n_common;
    if (n_common == 0) out->bitmap_data = nullptr;
    m.card[0] = tot;
    m.universe[0] = klen << 16;  // v2/src/multi_and.cu:446-449
    m.cstart[0] = 0;
    m.cstart[1] = n_common;
    m.kstart[0] = 0;
    m.kstart[1] = klen;
    m.nbm[0] = n_common;
    return CR_OK;
}

extern "C" int cr_batch_decompress(const cr_roaring_batch* batch, uint64_t* d_bitsets, uint64_t words_each,
                                   cr_stream_t stream)
{
    if (!batch) {
        set_error("cr_batch_decompress: invalid argument");
        return CR_ERR_INVALID;
    }
    if (batch->n_bitmaps == 0 || batch->total_containers == 0) return CR_OK;  // v2/src/decompress.cu:156
    if (!d_bitsets) {
        set_error("decompress_batch: device_bitsets is null");
        return CR_ERR_INVALID;
    }
    uint32_t max_u = 0;
    for (uint32_t b = 0; b < batch->n_bitmaps; ++b) max_u = std::max(max_u, batch->host_universe_sizes[b]);
    const uint64_t need = (static_cast<uint64_t>(max_u) + 63u) / 64u;
    if (words_each < need) {
        set_error("decompress_batch: words_each %llu < required %llu", static_cast<unsigned long long>(words_each),
                  static_cast<unsigned long long>(need));
        return CR_ERR_INVALID;
    }
    hipStream_t s = as_stream(stream);
    {
        CR_TIMED("bt_decompress", s);
        if (batch->run_pool_bytes == 0)
            bt_decompress<128, true><<<batch->total_containers, 128, 0, s>>>(*batch, d_bitsets, words_each);
        else
            bt_decompress<CV_NT, false><<<batch->total_containers, CV_NT, 0, s>>>(*batch, d_bitsets, words_each);
    }
    CR_LAUNCH_CHECK();
    return CR_OK;
}

extern "C" int cr_batch_contains(const cr_roaring_batch* batch, const uint32_t* d_bitmap_idx, uint32_t b,
                                 const uint32_t* d_ids, uint64_t n, uint8_t* d_out, cr_stream_t stream)
{
    if (!batch || (n && (!d_ids || !d_out))) {
        set_error("cr_batch_contains: invalid argument");
        return CR_ERR_INVALID;
    }
    if (n == 0) return CR_OK;
    hipStream_t s = as_stream(stream);
    GpuRoaringBatch B;
    std::memcpy(&B, batch, sizeof(B));
    {
        CR_TIMED("bt_contains", s);
        bt_contains<<<query_grid(n), 256, 0, s>>>(B, d_bitmap_idx, b, d_ids, n, d_out);
    }
    CR_LAUNCH_CHECK();
    return CR_OK;
}

extern "C" int cr_batch_view_contains(const cr_batch_view* view, const uint32_t* d_ids, uint64_t n, uint8_t* d_out,
                                      cr_stream_t stream)
{
    if (!view || (n && (!d_ids || !d_out))) {
        set_error("cr_batch_view_contains: invalid argument");
        return CR_ERR_INVALID;
    }
    if (n == 0) return CR_OK;
    hipStream_t s = as_stream(stream);
    GpuRoaringView v;
    std::memcpy(&v, view, sizeof(v));
    {
        CR_TIMED("bt_view_contains", s);
        bt_view_contains<<<query_grid(n), 256, 0, s>>>(v, d_ids, n, d_out);
    }
    CR_LAUNCH_CHECK();
    return CR_OK;
}

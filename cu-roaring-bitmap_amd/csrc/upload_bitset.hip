// upload_from_device_bitset / upload_from_bitset on gfx950.
//
// Semantics follow src/upload_ids.cu:606-893 (reference): 65536-bit chunks,
// every non-empty chunk becomes a BITMAP container (cards clamp 65536->0),
// complement when the popcount exceeds U/2 (strict), the inverted copy is
// masked only in the tail word U/32, max_key = last non-empty chunk,
// total_cardinality = the input's popcount.
//
// One read pass computes both the plain and the inverted popcount of every
// chunk, so the complement decision, the chunk->container map and all
// metadata are produced on the device and the call needs a single host sync.
#include <algorithm>

#include "internal.hpp"

namespace crimpl {

constexpr int BS_NT = 256;

struct BsTotals {
    uint32_t n_containers;
    uint32_t negated;
    uint32_t max_key;
    uint32_t done;  // planning workgroups finished
    unsigned long long total;  // popcount of the input
};

struct BsGeom {
    uint32_t n_words;
    uint32_t n_chunks;
    uint32_t tail_idx;   // word masked after inversion, or 0xFFFFFFFF
    uint32_t tail_mask;
    uint32_t universe;
};

__device__ __forceinline__ uint32_t load_word(const uint32_t* w, uint32_t i, uint32_t n) { return i < n ? w[i] : 0u; }

// Per chunk: popcount of the words and of their inversion (tail word masked,
// words past n_words are zero in both).  Workgroup 0 also clears the totals
// the planning workgroups accumulate.
__global__ __launch_bounds__(BS_NT) void bs_count(const uint32_t* __restrict__ words, BsGeom g, uint32_t* pc,
                                                  uint32_t* pci, BsTotals* tot)
{
    __shared__ uint32_t red[BS_NT / 64];
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        tot->n_containers = 0;
        tot->max_key = 0;
        tot->done = 0;
    }
    for (uint32_t c = blockIdx.x; c < g.n_chunks; c += gridDim.x) {
        const uint32_t base = c * 2048u;
        uint32_t a = 0, b = 0;
        if (base + 2048u <= g.n_words && (reinterpret_cast<uintptr_t>(words + base) & 15u) == 0) {
            const uint4* s4 = reinterpret_cast<const uint4*>(words + base);
            uint4 v[2];
#pragma unroll
            // Ordinary loads: the bitset (U/8 bytes, 128 MiB at 2^30) stays in
            // the Infinity Cache for bs_compact, which reads it again.
            for (int h = 0; h < 2; ++h) v[h] = s4[threadIdx.x + h * BS_NT];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t i0 = base + 4u * (threadIdx.x + h * BS_NT);
                const uint32_t x[4] = {v[h].x, v[h].y, v[h].z, v[h].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    a += __popc(x[q]);
                    b += (i0 + q == g.tail_idx) ? __popc(~x[q] & g.tail_mask) : 32u - __popc(x[q]);
                }
            }
        } else {
            for (uint32_t k = threadIdx.x; k < 2048u; k += BS_NT) {
                const uint32_t i = base + k;
                if (i < g.n_words) {
                    const uint32_t w = words[i];
                    a += __popc(w);
                    b += (i == g.tail_idx) ? __popc(~w & g.tail_mask) : 32u - __popc(w);
                }
            }
        }
        a = block_sum<BS_NT>(a, red);
        b = block_sum<BS_NT>(b, red);
        if (threadIdx.x == 0) {
            pc[c] = a;
            pci[c] = b;
        }
    }
}

// Planning: workgroup r takes the 1024 chunks of round r, [1024 r, 1024 r +
// 1024), one per thread.  Every workgroup sums the whole input's popcount
// (coalesced loads, eight rounds in flight, at most 64 rounds), which decides
// the negation (total > U/2, strict, src/upload_ids.cu:837); a chunk is kept
// iff its (plain or inverted) count is non-zero, and the kept chunks of the
// earlier rounds are counted again by every workgroup, so none waits for
// another.  Each writes its round of the chunk -> rank map and key_index, its
// kept chunks' keys/types/offsets/cards, and adds its count and its last kept
// chunk to `tot`; the last workgroup to finish (a counter, no waiting) writes
// the negation and the totals to `tot` and to the caller's pinned host slot.
__global__ __launch_bounds__(1024) void bs_plan(BsGeom g, const uint32_t* pc, const uint32_t* pci, uint32_t* cmap,
                                                uint16_t* keys, uint8_t* types, uint32_t* offsets, uint16_t* cards,
                                                uint16_t* key_index, BsTotals* tot, BsTotals* host)
{
    __shared__ unsigned long long wsum[16];
    __shared__ uint32_t lds[16], lds_i[16];
    __shared__ uint32_t s_last;
    __shared__ bool s_done;
    const uint32_t t = threadIdx.x, wave = t >> 6, lane = __lane_id();
    const uint32_t r = blockIdx.x, rounds = gridDim.x;
    // One pass of loads, sixteen rounds in flight a thread: the plain counts of
    // every round (their sum decides the negation) and both counts of the
    // rounds before r (kept chunks, plain and inverted), so nothing waits for
    // the negation before loading.
    const uint32_t c = r * 1024u + t;  // this thread's chunk: both counts
    const uint32_t own_p = c < g.n_chunks ? pc[c] : 0u, own_i = c < g.n_chunks ? pci[c] : 0u;
    unsigned long long part = 0;
    uint32_t bef_p = 0, bef_i = 0;
    for (uint32_t j0 = 0; j0 < rounds; j0 += 16) {
        uint32_t v[16], w[16];
#pragma unroll
        for (uint32_t q = 0; q < 16; ++q) {
            const uint32_t cq = (j0 + q) * 1024u + t;
            v[q] = cq < g.n_chunks ? pc[cq] : 0u;
            w[q] = j0 + q < r ? pci[cq] : 0u;  // rounds before r are whole
        }
#pragma unroll
        for (uint32_t q = 0; q < 16; ++q) {
            part += v[q];
            bef_p += j0 + q < r && v[q] != 0u ? 1u : 0u;
            bef_i += w[q] != 0u ? 1u : 0u;
        }
    }
    // One block reduction of the three: the total, and the kept chunks before
    // this round either way.
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        part += __shfl_xor(part, o, 64);
        bef_p += __shfl_xor(bef_p, o, 64);
        bef_i += __shfl_xor(bef_i, o, 64);
    }
    if (lane == 0) {
        wsum[wave] = part;
        lds[wave] = bef_p;
        lds_i[wave] = bef_i;
    }
    if (t == 0) s_last = 0;
    __syncthreads();
    unsigned long long total = 0;
    uint32_t base_p = 0, base_i = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
        total += wsum[w];
        base_p += lds[w];
        base_i += lds_i[w];
    }
    const bool negate = total > static_cast<unsigned long long>(g.universe / 2u);  // :837
    const uint32_t base = negate ? base_i : base_p;
    __syncthreads();  // lds is reused by the rank below
    const uint32_t v = negate ? own_i : own_p;
    const bool kept = v != 0u;
    uint32_t count;
    const uint32_t rank = base + block_flag_rank<1024>(kept, lds, count);
    uint32_t last = 0;
    if (kept) {
        cmap[c] = rank;
        keys[rank] = static_cast<uint16_t>(c);
        types[rank] = CR_BITMAP;
        offsets[rank] = rank * 8192u;
        cards[rank] = static_cast<uint16_t>(v > 65535u ? 0u : v);
        key_index[c] = static_cast<uint16_t>(rank);
        last = c;
    } else if (c < g.n_chunks) {
        cmap[c] = 0xFFFFFFFFu;
        key_index[c] = 0xFFFFu;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) last = max(last, static_cast<uint32_t>(__shfl_xor(last, o, 64)));
    if (lane == 0 && last) atomicMax(&s_last, last);
    __syncthreads();
    if (t == 0) {
        if (count) atomicAdd(&tot->n_containers, count);
        if (s_last) atomicMax(&tot->max_key, s_last);
        __threadfence();  // the updates above before the count of finished workgroups
        s_done = atomicAdd(&tot->done, 1u) == rounds - 1u;
    }
    __syncthreads();
    if (s_done && t == 0) {
        __threadfence();
        BsTotals res{};
        res.n_containers = __hip_atomic_load(&tot->n_containers, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        res.max_key = __hip_atomic_load(&tot->max_key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        res.negated = negate ? 1u : 0u;
        res.total = total;
        tot->negated = res.negated;
        tot->total = res.total;
        volatile BsTotals* h = host;
        h->n_containers = res.n_containers;
        h->negated = res.negated;
        h->max_key = res.max_key;
        h->total = res.total;
    }
}

__global__ __launch_bounds__(BS_NT) void bs_compact(const uint32_t* __restrict__ words, BsGeom g, const uint32_t* cmap,
                                                    const BsTotals* tot, uint64_t* __restrict__ pool)
{
    const bool negate = tot->negated != 0;
    for (uint32_t c = blockIdx.x; c < g.n_chunks; c += gridDim.x) {
        const uint32_t r = cmap[c];
        if (r == 0xFFFFFFFFu) continue;
        uint32_t* dst = reinterpret_cast<uint32_t*>(pool) + static_cast<uint64_t>(r) * 2048u;
        const uint32_t base = c * 2048u;
        const bool full = base + 2048u <= g.n_words;
        if (full && ((reinterpret_cast<uintptr_t>(words + base) & 15u) == 0)) {
            const uint4* s4 = reinterpret_cast<const uint4*>(words + base);
            uint4* d4 = reinterpret_cast<uint4*>(dst);
            uint4 v[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) v[h] = ld_stream(s4 + threadIdx.x + h * BS_NT);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if (negate) {
                    const uint32_t i0 = base + 4u * (threadIdx.x + h * BS_NT);
                    v[h] = make_uint4(~v[h].x, ~v[h].y, ~v[h].z, ~v[h].w);
                    if (i0 == g.tail_idx) v[h].x &= g.tail_mask;
                    if (i0 + 1 == g.tail_idx) v[h].y &= g.tail_mask;
                    if (i0 + 2 == g.tail_idx) v[h].z &= g.tail_mask;
                    if (i0 + 3 == g.tail_idx) v[h].w &= g.tail_mask;
                }
                st_stream(d4 + threadIdx.x + h * BS_NT, v[h]);
            }
        } else {
            for (uint32_t k = threadIdx.x; k < 2048u; k += BS_NT) {
                const uint32_t i = base + k;
                uint32_t w = 0;
                if (i < g.n_words) {
                    w = words[i];
                    if (negate) {
                        w = ~w;
                        if (i == g.tail_idx) w &= g.tail_mask;
                    }
                }
                dst[k] = w;
            }
        }
    }
}

static unsigned grid_cap(uint32_t n)
{
    const uint32_t cus = num_cus();
    return std::max(1u, std::min(n, static_cast<uint32_t>(cus) * 8u));
}

int upload_from_device_bitset_impl(const uint32_t* d_words, uint32_t n_words, uint32_t universe, hipStream_t s,
                                   cr_gpu_roaring* out)
{
    reset(out);
    out->universe_size = universe;
    if (n_words == 0) return CR_OK;  // src/upload_ids.cu:811-815
    BsGeom g{};
    g.n_words = n_words;
    g.n_chunks = static_cast<uint32_t>((static_cast<uint64_t>(n_words) + 2047u) / 2048u);
    if (g.n_chunks > 65536u) {
        set_error("upload_from_device_bitset: %u words exceed the 2^32-id key space", n_words);
        return CR_ERR_UNSUPPORTED;
    }
    g.universe = universe;
    const uint32_t tail_bits = universe % 32u;  // :851-858
    g.tail_idx = (tail_bits > 0 && universe / 32u < n_words) ? universe / 32u : 0xFFFFFFFFu;
    g.tail_mask = tail_bits ? ((1u << tail_bits) - 1u) : ~0u;

    Carver c;
    const size_t o_pc = c.add(4ull * g.n_chunks);
    const size_t o_pci = c.add(4ull * g.n_chunks);
    const size_t o_map = c.add(4ull * g.n_chunks);
    const size_t o_tot = c.add(sizeof(BsTotals));
    Scratch sc;
    CR_RET(sc.alloc(c.total, s));
    uint32_t* pc = sc.at<uint32_t>(o_pc);
    uint32_t* pci = sc.at<uint32_t>(o_pci);
    uint32_t* cmap = sc.at<uint32_t>(o_map);
    BsTotals* tot = sc.at<BsTotals>(o_tot);

    const OutLayout L = plan_out(g.n_chunks, g.n_chunks, static_cast<uint64_t>(g.n_chunks) * 1024u, 0, 0);
    CR_RET(alloc_out(out, L, g.n_chunks, g.n_chunks, static_cast<uint64_t>(g.n_chunks) * 1024u, 0, 0, s));

    {
        CR_TIMED("bs_count", s);
        bs_count<<<grid_cap(g.n_chunks), BS_NT, 0, s>>>(d_words, g, pc, pci, tot);
    }
    CR_LAUNCH_CHECK();
    HostSlotGuard hs;
    CR_RET(hs.acquire());
    {
        CR_TIMED("bs_plan", s);
        bs_plan<<<(g.n_chunks + 1023u) / 1024u, 1024, 0, s>>>(g, pc, pci, cmap, out->keys, out->types, out->offsets,
                                                               out->cardinalities, out->key_index, tot,
                                                               hs.dev<BsTotals>());
    }
    CR_LAUNCH_CHECK();
    {
        CR_TIMED("bs_compact", s);
        bs_compact<<<grid_cap(g.n_chunks), BS_NT, 0, s>>>(d_words, g, cmap, tot, out->bitmap_data);
    }
    CR_LAUNCH_CHECK();
    CR_RET(sync_stream(s));
    BsTotals h{};
    {
        const volatile BsTotals* hp = hs.host<BsTotals>();
        h.n_containers = hp->n_containers;
        h.negated = hp->negated;
        h.max_key = hp->max_key;
        h.total = hp->total;
    }
    out->negated = h.negated != 0;
    out->total_cardinality = h.total;  // logical count either way (:740)
    out->n_containers = h.n_containers;
    out->n_bitmap_containers = h.n_containers;
    if (h.n_containers == 0) {  // no key_index on an empty result (:747-750)
        free_async(out, s);
        out->universe_size = universe;
        out->negated = h.negated != 0;
        out->total_cardinality = h.total;
        return CR_OK;
    }
    out->max_key = h.max_key;
    return CR_OK;
}

}  // namespace crimpl

using namespace crimpl;

extern "C" int cr_upload_from_device_bitset(const uint32_t* d_words, uint32_t n_words, uint32_t universe_size,
                                            cr_stream_t stream, cr_gpu_roaring* out)
{
    if (!out || (n_words && !d_words)) {
        set_error("cr_upload_from_device_bitset: invalid argument");
        return CR_ERR_INVALID;
    }
    reset(out);
    return produced(upload_from_device_bitset_impl(d_words, n_words, universe_size, as_stream(stream), out), out,
                    as_stream(stream));
}

extern "C" int cr_upload_from_bitset(const uint32_t* host_words, uint32_t n_words, uint32_t universe_size,
                                     cr_stream_t stream, cr_gpu_roaring* out)
{
    if (!out || (n_words && !host_words)) {
        set_error("cr_upload_from_bitset: invalid argument");
        return CR_ERR_INVALID;
    }
    hipStream_t s = as_stream(stream);
    reset(out);
    if (n_words == 0) return produced(upload_from_device_bitset_impl(nullptr, 0, universe_size, s, out), out, s);
    Scratch sc;
    CR_RET(sc.alloc(static_cast<size_t>(n_words) * 4u, s));
    CR_RET(h2d_pageable(sc.ptr, host_words, static_cast<size_t>(n_words) * 4u, s));
    return produced(upload_from_device_bitset_impl(sc.at<uint32_t>(0), n_words, universe_size, s, out), out, s);
}

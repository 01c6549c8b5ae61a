// upload_from_ids on gfx950.
//
// Output semantics follow src/upload_ids.cu (reference): more than 1024 ids
// give an all-BITMAP result with keys sorted, offsets i*8192, cards clamped
// 65536->0, key_index sized from the universe (:171-295, :567-591); the
// complement is stored when the distinct count exceeds U/2 (:356-410); up to
// 1024 ids follow the threshold-aware small path (:421-561).
//
// The large path needs no global sort.  Ids are grouped by 16-key bucket
// (1 MiB of id space) inside 24576-id tiles, each bucket's 16 containers are
// built as 128 KiB of LDS bitmaps (the bit-set dedupes), and each container is
// written once:
//   tile_sort   read the ids once; counting-sort each tile by bucket in LDS and
//               stream it back to the tile's own slot as 20-bit fields (the id
//               within its bucket), with the tile's bucket starts in a small
//               table; max id per workgroup
//   build       one workgroup per bucket: read the bucket's run of every tile
//               (~24 fields, 60 bytes, at 2^30), LDS bit-set, popcount, write
//               each present key's container to pool slot `key`
//   rank        key ranks from the build's counts ->
//               keys/types/offsets/cards/key_index, totals, range error
// When the present keys are not a prefix of the key space, one more step
// moves the containers into a block of exactly n_containers slots.
#include <algorithm>
#include <vector>

#include "internal.hpp"
#include "tiles.hpp"

namespace crimpl {

// Key ranks after the build: workgroup r ranks the 1024 keys of round r,
// [1024 r, 1024 r + 1024), one per thread.  A key is present iff the build
// counted a bit in it.  The present keys of the earlier rounds are counted
// again by every workgroup (coalesced loads, eight rounds in flight, at most
// 63 rounds), so no workgroup waits for another.  Each writes its present
// keys' keys/types/offsets/cards at their ranks and its round of key_index
// (0xFFFF = absent), and adds its count and `moved` (a present key whose rank
// differs from the key: the build wrote container k to pool slot k) to `tot`;
// workgroup 0 adds the tile-sort workgroups' maximum id.  The last workgroup
// to finish (a counter, no waiting) writes the totals -- with the range error
// from the maximum id and the distinct count the build accumulated -- to `tot`
// and to the caller's pinned host slot.  When the build found every key of
// the universe present, the ranks are the keys and the build has written the
// metadata: workgroup 0 only writes the totals and the others return.
__global__ __launch_bounds__(1024) void ids_rank(IdsGeom g, const uint32_t* key_count, const uint32_t* gmax,
                                                 uint16_t* keys, uint8_t* types, uint32_t* offsets, uint16_t* cards,
                                                 uint16_t* key_index, IdsTotals* tot, IdsTotals* host, bool slotted)
{
    __shared__ uint32_t lds[16];
    __shared__ uint32_t s_max;
    __shared__ bool s_last;
    if (tot->absent == 0) {
        // Every key present: the ranks are the keys and the build wrote the
        // metadata; workgroup 0 writes the totals.
        if (blockIdx.x != 0) return;
        const uint32_t t = threadIdx.x;
        if (t == 0) s_max = 0;
        __syncthreads();
        uint32_t mx = 0;
        for (uint32_t i = t; i < g.G; i += 1024u) mx = max(mx, gmax[i]);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) mx = max(mx, static_cast<uint32_t>(__shfl_xor(mx, o, 64)));
        if (__lane_id() == 0) atomicMax(&s_max, mx);
        __syncthreads();
        if (t == 0) {
            IdsTotals res{};
            res.n_containers = g.K;
            res.max_id = s_max;
            res.err = (s_max >> 16) > g.K - 1u ? 1u : 0u;
            res.moved = 0;
            res.total = tot->total;
            tot->n_containers = res.n_containers;
            tot->max_id = res.max_id;
            tot->err = res.err;
            volatile IdsTotals* h = host;
            h->n_containers = res.n_containers;
            h->err = res.err;
            h->max_id = res.max_id;
            h->moved = res.moved;
            h->total = res.total;
        }
        return;
    }
    const uint32_t t = threadIdx.x, lane = __lane_id();
    const uint32_t r = blockIdx.x;
    if (t == 0) s_max = 0;
    // Rounds before r are whole (only the last round can be partial).
    uint32_t before = 0;
    for (uint32_t j0 = 0; j0 < r; j0 += 8) {
        uint32_t c[8];
#pragma unroll
        for (uint32_t q = 0; q < 8; ++q) c[q] = j0 + q < r ? key_count[(j0 + q) * 1024u + t] : 0u;
#pragma unroll
        for (uint32_t q = 0; q < 8; ++q) before += c[q] != 0u ? 1u : 0u;
    }
    const uint32_t base = block_sum<1024>(before, lds);
    const uint32_t k = r * 1024u + t;
    const uint32_t c = k < g.K ? key_count[k] : 0u;
    const bool present = c != 0u;
    uint32_t count;
    const uint32_t rank = base + block_flag_rank<1024>(present, lds, count);
    bool moved = false;
    if (present) {
        keys[rank] = static_cast<uint16_t>(k);
        types[rank] = CR_BITMAP;
        offsets[rank] = rank * 8192u;
        cards[rank] = static_cast<uint16_t>(c > 65535u ? 0u : c);  // 65536 stored as 0
        key_index[k] = static_cast<uint16_t>(rank);
        moved = !slotted && rank != k;  // slotted: the build wrote the container at its rank
    } else if (k < g.K) {
        key_index[k] = 0xFFFFu;
    }
    const bool any_moved = __syncthreads_or(moved) != 0;  // also: s_max is initialised
    if (r == 0) {
        uint32_t mx = 0;
        for (uint32_t i = t; i < g.G; i += 1024u) mx = max(mx, gmax[i]);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) mx = max(mx, static_cast<uint32_t>(__shfl_xor(mx, o, 64)));
        if (lane == 0) atomicMax(&s_max, mx);
        __syncthreads();
    }
    if (t == 0) {
        if (count) atomicAdd(&tot->n_containers, count);
        if (any_moved) atomicOr(&tot->moved, 1u);
        if (r == 0) atomicMax(&tot->max_id, s_max);
        __threadfence();  // the updates above before the count of finished workgroups
        s_last = atomicAdd(&tot->done, 1u) == gridDim.x - 1u;
    }
    __syncthreads();
    if (s_last && t == 0) {
        __threadfence();
        IdsTotals res;
        res.n_containers = __hip_atomic_load(&tot->n_containers, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        res.max_id = __hip_atomic_load(&tot->max_id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        res.moved = __hip_atomic_load(&tot->moved, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        res.total = __hip_atomic_load(&tot->total, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        res.err = (res.max_id >> 16) > g.K - 1u ? 1u : 0u;
        tot->err = res.err;
        volatile IdsTotals* h = host;
        h->n_containers = res.n_containers;
        h->err = res.err;
        h->max_id = res.max_id;
        h->moved = res.moved;
        h->total = res.total;
    }
}

// Fewer ids than keys (n < K): at most n containers, so the pool holds n
// slots, not K, and each container is built straight at its rank.  The keys
// present among the ids are marked as bits (an id whose key is past max_key is
// left to the error check), then ranked into key_index (0xFFFF: absent), which
// the build reads as its slot map and ids_rank rewrites with the same values.
__global__ __launch_bounds__(256) void ids_presence(const uint32_t* __restrict__ ids, uint32_t n, uint32_t K,
                                                    uint32_t* bits)
{
    for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < n; i += gridDim.x * 256u) {
        const uint32_t k = ids[i] >> 16;
        if (k < K) atomicOr(&bits[k >> 5], 1u << (k & 31u));
    }
}

__global__ __launch_bounds__(1024) void ids_slots(const uint32_t* __restrict__ bits, uint32_t K, uint16_t* key_index)
{
    __shared__ uint32_t lds[16];
    const uint32_t t = threadIdx.x;  // keys [64 t, 64 t + 64): words 2 t, 2 t + 1
    const uint32_t nw = (K + 31u) / 32u;
    const uint32_t w0 = 2u * t < nw ? bits[2u * t] : 0u, w1 = 2u * t + 1u < nw ? bits[2u * t + 1u] : 0u;
    uint32_t total;
    uint32_t r = block_excl_scan<1024>(static_cast<uint32_t>(__popc(w0) + __popc(w1)), lds, total);
    if (64u * t >= K) return;
    // The 64 entries as 32 packed pairs; a whole row goes out as eight
    // 16-byte stores (key_index is 256-byte aligned), the last partial one
    // entry by entry.
    uint32_t pk[32];
#pragma unroll
    for (uint32_t j = 0; j < 64u; ++j) {
        const bool present = ((j < 32u ? w0 >> j : w1 >> (j - 32u)) & 1u) != 0u;
        const uint32_t v = present ? r : 0xFFFFu;
        r += present ? 1u : 0u;
        if (j & 1u)
            pk[j >> 1] |= v << 16;
        else
            pk[j >> 1] = v;
    }
    if (64u * t + 64u <= K) {
        uint4* dst = reinterpret_cast<uint4*>(key_index + 64u * t);
#pragma unroll
        for (uint32_t q = 0; q < 8u; ++q) dst[q] = make_uint4(pk[4 * q], pk[4 * q + 1], pk[4 * q + 2], pk[4 * q + 3]);
    } else {
#pragma unroll
        for (uint32_t j = 0; j < 64u; ++j)
            if (64u * t + j < K) key_index[64u * t + j] = static_cast<uint16_t>(pk[j >> 1] >> ((j & 1u) * 16u));
    }
}

// Pool compaction when present keys are not a prefix: container i moves from
// slot keys[i] of the key-addressed pool to slot i.  One wave per container.
__global__ __launch_bounds__(256) void ids_gather_pool(const uint16_t* keys, uint32_t n_c,
                                                       const uint64_t* __restrict__ src, uint64_t* __restrict__ dst)
{
    const uint32_t i = (blockIdx.x * 256u + threadIdx.x) >> 6;
    const uint32_t lane = __lane_id();
    if (i >= n_c) return;
    const uint4* s4 = reinterpret_cast<const uint4*>(src + static_cast<uint64_t>(keys[i]) * 1024u);
    uint4* d4 = reinterpret_cast<uint4*>(dst + static_cast<uint64_t>(i) * 1024u);
    uint4 x[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) x[k] = ld_stream(s4 + lane + 64 * k);
#pragma unroll
    for (int k = 0; k < 8; ++k) st_stream(d4 + lane + 64 * k, x[k]);
}

// A bucket's 16 containers are 16 x 2048 u32 LDS words (128 KiB), filled from
// the bucket's run in every tile.  The build is persistent: up to one
// workgroup per CU, and XCD x's workgroups (blockIdx % 8 == x) share the
// contiguous bucket range [x * per, (x + 1) * per) -- neighbouring buckets,
// whose runs share the cache line at their boundary in every tile, are built
// close in time on one XCD.  The group's first round is static (its i-th
// workgroup builds the range's i-th bucket); the rest of the range goes out
// through a ticket counter, heaviest bucket first, so a skewed input does not
// leave its heaviest buckets to the end (list scheduling, longest first).
// The order comes from the tile sort's per-workgroup counts: each workgroup
// sums them for the ticketed buckets while its first bucket's run bounds
// load, and ranks the buckets by count in BUILD_LEVELS classes of the
// largest, ties in bucket order (equal buckets keep the contiguous order).
// Measured on 100M ids at 2^30 (kernel time, one box): clustered runs 0.157
// -> 0.123 ms, against one workgroup per bucket in bucket order; uniform ids
// unchanged (0.124-0.127 ms).
// Normal mode writes each present key's container to pool slot `key`, every
// key's distinct count, and the metadata as if ranks were keys (right when
// every key is present; ids_rank rewrites it otherwise, told by `absent`);
// complement mode writes ~bits masked to [0, U) at the key_index rank of keys
// whose complement is non-empty, with their cards.

// Normal mode's metadata outputs: with every key present the ranks are the
// keys, so the build writes keys/types/offsets/cards/key_index itself (and
// ids_rank only the totals); otherwise ids_rank rewrites them in rank order.
// The arrays hold min(K, n) entries, so the build is handed them (non-null
// `keys`) only when n >= K: with fewer ids not every key can be present, and
// a write at index `key` could land past the arrays.
struct BuildMeta {
    uint16_t* keys;
    uint8_t* types;
    uint32_t* offsets;
    uint16_t* cards;
    uint16_t* key_index;
};

constexpr uint32_t BUILD_LEVELS = 16;  // bucket weight classes of the build order

__global__ __launch_bounds__(BUILD_NT) void ids_build(const uint32_t* __restrict__ part,
                                                      const uint16_t* __restrict__ tab, IdsGeom g,
                                                      const uint32_t* __restrict__ wg_count, uint32_t universe,
                                                      bool complement, const uint16_t* key_index,
                                                      uint64_t* __restrict__ pool, uint16_t* cards,
                                                      uint32_t* key_count, IdsTotals* tot, BuildMeta m)
{
    __shared__ alignas(16) uint32_t bits[BK_KEYS * 2048u];  // 128 KiB of the CU's 160 KiB LDS
    constexpr uint32_t MAX_PER = MAX_BUCKETS / 8;
    __shared__ uint32_t wt[MAX_PER], rank[MAX_PER], order[MAX_PER];
    __shared__ uint32_t wave_pc[BUILD_WAVES];
    __shared__ uint32_t s_next, s_wmax;
    __shared__ GroupQueue queue;
    __shared__ uint32_t desc[BUILD_WAVES * DESC_CAP];
    const uint32_t t = threadIdx.x;
    const uint32_t wave = t >> 6;
    const uint32_t x = blockIdx.x % 8, slot = blockIdx.x / 8;
    const uint32_t per = build_per_xcd(g.NB);
    const uint32_t lo = x * per;
    if (lo >= g.NB) return;  // the whole workgroup
    const uint32_t nx = min(per, g.NB - lo);
    // The group's first round is static (workgroup `slot` builds bucket
    // lo + slot); the other nt buckets, lo + S0 + j, are taken by ticket in
    // the order `order` computes during the first bucket.
    const uint32_t S0 = min(gridDim.x / 8, nx);
    const uint32_t nt = nx - S0;

    // order[k] = j for the k-th heaviest of buckets lo + S0 + j: the tile
    // sort's per-workgroup counts summed (R threads a bucket, each over every
    // R-th row), put in BUILD_LEVELS classes of the largest, and ranked by
    // (class descending, bucket ascending).
    auto compute_order = [&] {
        if (nt == 0) return;  // the same in every thread
        const uint32_t base = lo + S0;
        const uint32_t R = BUILD_NT / nt;  // >= 2: nt <= MAX_PER = 512
        if (t < nt) wt[t] = 0, rank[t] = 0;
        if (t == 0) s_wmax = 0;
        uint32_t sum = 0;
        if (t < R * nt) {
            const uint32_t j = t % nt;
            for (uint32_t w0 = t / nt; w0 < g.G; w0 += 32u * R) {  // 32 loads in flight
                uint32_t c[32];
#pragma unroll
                for (uint32_t k = 0; k < 32u; ++k) {
                    const uint32_t w = w0 + k * R;
                    c[k] = w < g.G ? wg_count[static_cast<uint64_t>(w) * g.NB + base + j] : 0u;
                }
#pragma unroll
                for (uint32_t k = 0; k < 32u; ++k) sum += c[k];
            }
        }
        __syncthreads();  // wt, rank, s_wmax cleared
        if (t < R * nt) atomicAdd(&wt[t % nt], sum);
        __syncthreads();
        if (t < nt) atomicMax(&s_wmax, wt[t]);
        __syncthreads();
        if (t < nt)  // the class, once a bucket (in place of its total)
            wt[t] = static_cast<uint32_t>(static_cast<uint64_t>(wt[t]) * BUILD_LEVELS /
                                          (static_cast<uint64_t>(s_wmax) + 1u));
        __syncthreads();
        if (t < R * nt) {
            const uint32_t j = t % nt, p = t / nt;
            const uint32_t lj = wt[j];
            uint32_t r = 0;
            for (uint32_t i = p * nt / R; i < (p + 1) * nt / R; ++i) {
                const uint32_t li = wt[i];
                r += (li > lj || (li == lj && i < j)) ? 1u : 0u;
            }
            atomicAdd(&rank[j], r);
        }
        __syncthreads();
        if (t < nt) order[rank[t]] = t;
    };

    // Builds bucket b and returns the next one (g.NB: none); the first call
    // (FIRST) also computes the order while its run bounds load.
    auto build_bucket = [&](uint32_t b, auto first) -> uint32_t {
        // The lane index, opaque to the compiler inside each bucket: values
        // derived from it are recomputed per bucket rather than held in
        // registers across the whole loop.
        uint32_t lane = __lane_id();
        asm volatile("" : "+v"(lane));
        walk_groups<true>(part, tab, g, b, wave, lane, queue, desc,
                    [&] {
                        for (uint32_t i = t; i < BK_KEYS * 512u; i += BUILD_NT)
                            reinterpret_cast<uint4*>(bits)[i] = make_uint4(0, 0, 0, 0);
                        if constexpr (decltype(first)::value) compute_order();
                    },
                    [&](uint32_t, uint32_t, uint32_t n, const uint32_t (&f)[8]) {
                        // An empty slot sets nothing (its lanes would all hit one
                        // group's words).  When no lane of the wave holds a partial
                        // group (only runs of fewer than 8 fields make one), every
                        // field is set; otherwise the fields past a run OR in
                        // nothing (no branch per field).
                        const bool whole = __ballot(n - 1u < 7u) == 0ull;  // wave-uniform
                        if (n == 0u) return;
                        if (whole) {
#pragma unroll
                            for (uint32_t k = 0; k < 8u; ++k) {
                                const uint32_t F = f[k] & FIELD_MASK;  // key-in-bucket << 16 | low 16 bits
                                atomicOr(&bits[F >> 5], 1u << (F & 31u));
                            }
                        } else {
                            const uint32_t live = (1u << n) - 1u;  // bit k: field k is the run's
#pragma unroll
                            for (uint32_t k = 0; k < 8u; ++k) {
                                const uint32_t F = f[k] & FIELD_MASK;
                                atomicOr(&bits[F >> 5], ((live >> k) & 1u) << (F & 31u));
                            }
                        }
                    });
        __syncthreads();
        uint32_t nxt = 0;
        if (t == 0) nxt = atomicAdd(&tot->ticket[x], 1u);  // the next bucket, fetched during the write-out
        const uint32_t c = wave;  // wave c owns container c of the bucket
        const uint32_t key = b * BK_KEYS + c;
        uint32_t pc = 0;
        if (key < g.K) {
            uint32_t* cb = bits + c * 2048u;
            uint32_t valid_words = 2048, tail_mask = ~0u;
            if (complement) {
                const uint64_t valid =
                    min<uint64_t>(65536u, static_cast<uint64_t>(universe) - static_cast<uint64_t>(key) * 65536u);
                valid_words = static_cast<uint32_t>(valid >> 5);
                tail_mask = (valid & 31u) ? ((1u << (valid & 31u)) - 1u) : 0u;
            }
            // The container is read from LDS once, as eight 16-byte vectors a lane.
            uint4 v[8];
            const uint4* src = reinterpret_cast<const uint4*>(cb);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                v[q] = src[lane + 64 * q];
                if (complement) {
                    const uint32_t i0 = 4u * (lane + 64u * q);
                    uint32_t xw[4] = {~v[q].x, ~v[q].y, ~v[q].z, ~v[q].w};
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (i0 + e >= valid_words) xw[e] = (i0 + e == valid_words) ? (xw[e] & tail_mask) : 0u;
                    v[q] = make_uint4(xw[0], xw[1], xw[2], xw[3]);
                }
                pc += __popc(v[q].x) + __popc(v[q].y) + __popc(v[q].z) + __popc(v[q].w);
            }
            pc = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(wave_incl_scan(pc)), 63));
            if (!complement && lane == 0) {
                key_count[key] = pc;
                if (pc != 0 && m.keys != nullptr) {
                    m.keys[key] = static_cast<uint16_t>(key);
                    m.types[key] = CR_BITMAP;
                    m.offsets[key] = key * 8192u;
                    m.cards[key] = static_cast<uint16_t>(pc > 65535u ? 0u : pc);  // 65536 stored as 0
                    m.key_index[key] = static_cast<uint16_t>(key);
                }
            }
            if (pc != 0) {
                // the key's rank when a slot map is given (complement mode, or
                // fewer ids than keys), else the key itself
                const uint32_t slot = key_index != nullptr ? key_index[key] : key;
                uint4* dst = reinterpret_cast<uint4*>(pool + static_cast<uint64_t>(slot) * 1024u);
#pragma unroll
                for (int q = 0; q < 8; ++q) st_stream(dst + lane + 64 * q, v[q]);
                if (complement && lane == 0) cards[slot] = static_cast<uint16_t>(pc > 65535u ? 0u : pc);
            }
        }
        if (lane == 0) wave_pc[c] = pc;
        __syncthreads();  // also: every wave's reads of the image are done before the next bucket clears it
        if (t == 0) {  // device atomics without a return
            unsigned long long sum = 0;
            bool absent = false;
            for (uint32_t i = 0; i < BUILD_WAVES; ++i) {
                sum += wave_pc[i];
                absent |= b * BK_KEYS + i < g.K && wave_pc[i] == 0;
            }
            if (sum) atomicAdd(&tot->total, sum);
            if (!complement && absent) atomicAdd(&tot->absent, 1u);
            s_next = nxt < nt ? lo + S0 + order[nxt] : g.NB;
        }
        __syncthreads();
        return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(s_next));
    };

    // Workgroups past the group's first round (only when it has no ticketed
    // buckets: nt == 0) leave at once.
    uint32_t b = slot < nx ? lo + slot : g.NB;
    if (b < g.NB) b = build_bucket(b, std::true_type{});
    while (b < g.NB) b = build_bucket(b, std::false_type{});
}

// Complement key plan: key k is stored iff its complement within [0, U) is
// non-empty.  Writes keys/types/offsets/key_index and the container count.
__global__ __launch_bounds__(1024) void ids_keyscan_complement(IdsGeom g, uint32_t universe, const uint32_t* key_count,
                                                               uint16_t* keys, uint8_t* types, uint32_t* offsets,
                                                               uint16_t* key_index, IdsTotals* tot)
{
    __shared__ uint32_t lds[16];
    const uint32_t t = threadIdx.x;
    uint64_t present = 0;
    for (uint32_t kk = 0; kk < 64; ++kk) {
        const uint32_t key = 64 * t + kk;
        if (key >= g.K) break;
        const uint64_t valid = min<uint64_t>(65536u, static_cast<uint64_t>(universe) - static_cast<uint64_t>(key) * 65536u);
        if (valid > key_count[key]) present |= 1ull << kk;
    }
    uint32_t total;
    uint32_t rank = block_excl_scan<1024>(static_cast<uint32_t>(__popcll(present)), lds, total);
    for (uint32_t kk = 0; kk < 64; ++kk) {
        const uint32_t key = 64 * t + kk;
        if (key >= g.K) break;
        if ((present >> kk) & 1u) {
            keys[rank] = static_cast<uint16_t>(key);
            types[rank] = CR_BITMAP;
            offsets[rank] = rank * 8192u;
            key_index[key] = static_cast<uint16_t>(rank);
            ++rank;
        } else {
            key_index[key] = 0xFFFFu;
        }
    }
    if (t == 0) {
        tot->n_containers = total;
        tot->total = 0;
    }
    if (t < 8) tot->ticket[t] = 0;  // the complement build takes the buckets again
}

// ---- small path (n <= 1024), src/upload_ids.cu:421-561 --------------------
constexpr uint32_t SMALL_MAX = 1024;

struct SmallPlan {
    uint32_t n_vals;        // stored values (complement when negated)
    uint32_t n_containers;
    uint32_t n_bitmap, n_array, arr_elems;
    uint32_t total;         // distinct ids
    uint32_t negated;
    uint32_t max_key;       // last stored key
    uint32_t vals[2 * SMALL_MAX];
    uint32_t cstart[2 * SMALL_MAX + 1];
    uint32_t bslot[2 * SMALL_MAX];  // bitmap pool slot of a bitmap container (ids_small_write fills it)
};

__global__ __launch_bounds__(1024) void ids_small_plan(const uint32_t* ids, uint32_t n, uint32_t universe, uint32_t thr,
                                                       SmallPlan* plan)
{
    __shared__ uint32_t v[SMALL_MAX];
    __shared__ uint32_t u[2 * SMALL_MAX];
    __shared__ uint32_t lds[16];
    __shared__ uint32_t s_m, s_nv;
    const uint32_t t = threadIdx.x;
    v[t] = t < n ? ids[t] : 0xFFFFFFFFu;
    __syncthreads();
    for (uint32_t k = 2; k <= SMALL_MAX; k <<= 1) {  // bitonic sort
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            const uint32_t p = t ^ j;
            if (p > t) {
                const uint32_t a = v[t], b = v[p];
                const bool up = (t & k) == 0;
                if ((a > b) == up) {
                    v[t] = b;
                    v[p] = a;
                }
            }
            __syncthreads();
        }
    }
    const bool first = t < n && (t == 0 || v[t] != v[t - 1]);
    uint32_t m;
    const uint32_t r = block_flag_rank<1024>(first, lds, m);
    if (first) u[r] = v[t];
    if (t == 0) s_m = m;
    __syncthreads();
    const bool negate = static_cast<uint64_t>(m) > static_cast<uint64_t>(universe) / 2u;  // :437
    uint32_t nv = m;
    if (negate) {
        // universe < 2*m <= 2048: complement over [0, U) by binary search in u[0, m).
        uint32_t cand[2];
        bool keepc[2];
        for (int q = 0; q < 2; ++q) {
            const uint32_t x = 2 * t + q;
            cand[q] = x;
            bool in = false;
            if (x < universe) {
                uint32_t lo = 0, hi = m;
                while (lo < hi) {
                    const uint32_t mid = (lo + hi) >> 1;
                    if (u[mid] < x)
                        lo = mid + 1;
                    else
                        hi = mid;
                }
                in = lo < m && u[lo] == x;
            }
            keepc[q] = x < universe && !in;
        }
        uint32_t tot;
        uint32_t pos = block_excl_scan<1024>(static_cast<uint32_t>(keepc[0]) + keepc[1], lds, tot);
        __syncthreads();  // every lane has read u[] before it is overwritten
        for (int q = 0; q < 2; ++q)
            if (keepc[q]) u[pos++] = cand[q];
        nv = tot;
        __syncthreads();
    }
    if (t == 0) s_nv = nv;
    __syncthreads();
    nv = s_nv;
    for (uint32_t i = t; i < nv; i += 1024) plan->vals[i] = u[i];
    // container boundaries: value i starts a container if its key differs
    uint32_t nstart = 0;
    bool st[2];
    for (int q = 0; q < 2; ++q) {
        const uint32_t i = 2 * t + q;
        st[q] = i < nv && (i == 0 || (u[i] >> 16) != (u[i - 1] >> 16));
        nstart += st[q];
    }
    uint32_t nc;
    uint32_t cpos = block_excl_scan<1024>(nstart, lds, nc);
    for (int q = 0; q < 2; ++q)
        if (st[q]) plan->cstart[cpos++] = 2 * t + q;
    __syncthreads();
    if (t == 0) {
        plan->cstart[nc] = nv;
        plan->n_vals = nv;
        plan->n_containers = nc;
        plan->total = s_m;
        plan->negated = negate ? 1u : 0u;
        plan->max_key = nv ? (u[nv - 1] >> 16) : 0u;
    }
    __threadfence_block();
    __syncthreads();
    // types and pool sizes (threshold rule :493)
    uint32_t nb = 0, na = 0, ae = 0;
    for (uint32_t c = t; c < nc; c += 1024) {
        const uint32_t card = plan->cstart[c + 1] - plan->cstart[c];
        if (card > thr)
            ++nb;
        else {
            ++na;
            ae += card;
        }
    }
    uint32_t s0, s1, s2;
    block_excl_scan<1024>(nb, lds, s0);
    block_excl_scan<1024>(na, lds, s1);
    block_excl_scan<1024>(ae, lds, s2);
    if (t == 0) {
        plan->n_bitmap = s0;
        plan->n_array = s1;
        plan->arr_elems = s2;
    }
}

// Single workgroup: containers are laid out in key order; bitmap containers
// take consecutive 8 KiB slots, array containers consecutive ranges.
__global__ __launch_bounds__(1024) void ids_small_write(SmallPlan* plan, uint32_t thr, uint16_t* keys,
                                                        uint8_t* types, uint32_t* offsets, uint16_t* cards,
                                                        uint64_t* bmp, uint16_t* arr, uint16_t* key_index,
                                                        uint32_t kidx_len)
{
    __shared__ uint32_t s_bslot[2 * SMALL_MAX + 1], s_aoff[2 * SMALL_MAX + 1];
    __shared__ uint32_t lds[16];
    const uint32_t t = threadIdx.x;
    const uint32_t nc = plan->n_containers;
    {  // slot prefixes: containers 2t and 2t+1
        uint32_t card[2], nb = 0, ae = 0;
        for (int q = 0; q < 2; ++q) {
            const uint32_t c = 2 * t + q;
            card[q] = c < nc ? plan->cstart[c + 1] - plan->cstart[c] : 0u;
            if (c < nc) {
                if (card[q] > thr)
                    ++nb;
                else
                    ae += card[q];
            }
        }
        uint32_t tb, ta;
        uint32_t bs = block_excl_scan<1024>(nb, lds, tb);
        uint32_t ao = block_excl_scan<1024>(ae, lds, ta);
        for (int q = 0; q < 2; ++q) {
            const uint32_t c = 2 * t + q;
            if (c >= nc) continue;
            s_bslot[c] = bs;
            s_aoff[c] = ao;
            if (card[q] > thr)
                ++bs;
            else
                ao += card[q];
        }
    }
    for (uint32_t i = t; i < kidx_len; i += 1024) key_index[i] = 0xFFFFu;
    __syncthreads();
    for (uint32_t c = t; c < nc; c += 1024) {
        const uint32_t s = plan->cstart[c], e = plan->cstart[c + 1], card = e - s;
        const uint32_t key = plan->vals[s] >> 16;
        keys[c] = static_cast<uint16_t>(key);
        cards[c] = static_cast<uint16_t>(card > 65535u ? 0u : card);
        key_index[key] = static_cast<uint16_t>(c);
        if (card > thr) {
            types[c] = CR_BITMAP;
            offsets[c] = s_bslot[c] * 8192u;
            plan->bslot[c] = s_bslot[c];
        } else {
            types[c] = CR_ARRAY;
            offsets[c] = s_aoff[c] * 2u;
            for (uint32_t i = s; i < e; ++i) arr[s_aoff[c] + (i - s)] = static_cast<uint16_t>(plan->vals[i]);
        }
    }
}

// The bitmap containers of the small path: one workgroup per container builds
// its 8 KiB image in LDS from the container's values and writes it once with
// 16-byte stores (containers that are arrays leave at once).
__global__ __launch_bounds__(256) void ids_small_bitmaps(const SmallPlan* __restrict__ plan, uint32_t thr,
                                                         uint64_t* __restrict__ bmp)
{
    __shared__ alignas(16) uint32_t img[2048];
    const uint32_t c = blockIdx.x, t = threadIdx.x;
    const uint32_t s = plan->cstart[c], e = plan->cstart[c + 1];
    if (e - s <= thr) return;  // the same test for the whole workgroup
    uint4* img4 = reinterpret_cast<uint4*>(img);
    img4[t] = make_uint4(0, 0, 0, 0);
    img4[t + 256] = make_uint4(0, 0, 0, 0);
    __syncthreads();
    for (uint32_t i = s + t; i < e; i += 256u) {
        const uint32_t low = plan->vals[i] & 0xFFFFu;
        atomicOr(&img[low >> 5], 1u << (low & 31u));
    }
    __syncthreads();
    uint4* dst = reinterpret_cast<uint4*>(bmp + static_cast<uint64_t>(plan->bslot[c]) * 1024u);
    dst[t] = img4[t];
    dst[t + 256] = img4[t + 256];
}

static int small_upload(const uint32_t* d_ids, uint32_t n, uint32_t universe, uint32_t thr, hipStream_t s,
                        cr_gpu_roaring* out)
{
    Scratch sc;
    CR_RET(sc.alloc(sizeof(SmallPlan), s));
    SmallPlan* plan = sc.at<SmallPlan>(0);
    {
        CR_TIMED("ids_small_plan", s);
        ids_small_plan<<<1, 1024, 0, s>>>(d_ids, n, universe, thr, plan);
    }
    CR_LAUNCH_CHECK();
    uint32_t hdr[8];
    CR_RET(read_back(hdr, plan, sizeof(hdr), s));
    const uint32_t nc = hdr[1], n_bitmap = hdr[2], n_array = hdr[3], arr_elems = hdr[4];
    out->total_cardinality = hdr[5];
    out->negated = hdr[6] != 0;
    if (nc == 0) return CR_OK;  // src/upload_ids.cu:454-456
    const uint32_t max_key = hdr[7];
    const uint64_t kidx_len = static_cast<uint64_t>(max_key) + 1u;  // last key (:547)
    const uint64_t bmp_words = static_cast<uint64_t>(n_bitmap) * 1024u;
    const OutLayout L = plan_out(nc, kidx_len, bmp_words, arr_elems, 0);
    CR_RET(alloc_out(out, L, nc, kidx_len, bmp_words, arr_elems, 0, s));
    out->n_containers = nc;
    out->n_bitmap_containers = n_bitmap;
    out->n_array_containers = n_array;
    out->array_pool_bytes = arr_elems ? arr_elems * 2u : 0u;
    out->max_key = max_key;
    {
        CR_TIMED("ids_small_write", s);
        ids_small_write<<<1, 1024, 0, s>>>(plan, thr, out->keys, out->types, out->offsets, out->cardinalities,
                                           out->bitmap_data, out->array_data, out->key_index,
                                           static_cast<uint32_t>(kidx_len));
    }
    CR_LAUNCH_CHECK();
    if (n_bitmap) {
        CR_TIMED("ids_small_bitmaps", s);
        ids_small_bitmaps<<<nc, 256, 0, s>>>(plan, thr, out->bitmap_data);
    }
    CR_LAUNCH_CHECK();
    CR_RET(sync_stream(s));
    return CR_OK;
}

// u32 id counts: the tiles' word offsets (group_word) stay below 2^32.
static_assert((0xFFFFFFFFull + TILE - 1) / TILE <= 0xFFFFFFFFull / TILE_WORDS, "tile count bound");

static int large_upload(const uint32_t* d_ids, uint32_t n, uint32_t universe, hipStream_t s, cr_gpu_roaring* out)
{
    if (universe == 0) {
        set_error("upload_from_ids: universe_size 0 with %u ids (the reference's complement underflows)", n);
        return CR_ERR_INVALID;
    }
    uint32_t max_key32 = (universe - 1u) >> 16;  // src/upload_ids.cu:274-278
    if (max_key32 > 0xFFFFu) max_key32 = 0xFFFFu;
    IdsGeom g{};
    g.n = n;
    g.K = max_key32 + 1u;
    g.NB = (g.K + BK_KEYS - 1) / BK_KEYS;
    g.n_tiles = static_cast<uint32_t>((static_cast<uint64_t>(n) + TILE - 1) / TILE);
    g.G = std::max<uint32_t>(1, std::min<uint32_t>(num_cus(), (g.n_tiles + TB - 1) / TB));  // blocks of TB tiles
    g.vec = (reinterpret_cast<uintptr_t>(d_ids) & 15u) == 0;

    Carver c;
    const size_t o_gmax = c.add(sizeof(uint32_t) * g.G);
    const size_t o_kc = c.add(sizeof(uint32_t) * g.K);
    const size_t o_tot = c.add(sizeof(IdsTotals));
    const size_t o_tab =
        c.add(sizeof(uint16_t) * static_cast<uint64_t>((g.n_tiles + TB - 1) / TB) * TB * (g.NB + 1));
    // Whole tiles (a partial last tile is padded) + the build's window overrun.
    // the build's field groups read up to 5 words past a group's first: slack past the last tile
    const size_t o_part = c.add(sizeof(uint32_t) * (static_cast<uint64_t>(g.n_tiles) * TILE_WORDS + 8));
    const size_t o_wgc = c.add(sizeof(uint32_t) * static_cast<uint64_t>(g.G) * g.NB);
    const size_t o_pres = c.add(sizeof(uint32_t) * 2048u);  // key presence bits (fewer ids than keys)
    Scratch sc;
    CR_RET(sc.alloc(c.total, s));
    uint32_t* gmax = sc.at<uint32_t>(o_gmax);
    uint32_t* key_count = sc.at<uint32_t>(o_kc);
    IdsTotals* tot = sc.at<IdsTotals>(o_tot);
    uint16_t* tab = sc.at<uint16_t>(o_tab);
    uint32_t* part = sc.at<uint32_t>(o_part);
    uint32_t* wg_count = sc.at<uint32_t>(o_wgc);

    // Containers <= min(keys, ids) bounds the metadata.  With an id for every
    // key possible (n >= K) the pool is addressed by key (slot k holds key
    // k's container) until the ranks are known; with fewer ids than keys the
    // ranks come first and the pool holds n slots (src/upload_ids.cu:243-262
    // sizes it by the container count too).
    const uint64_t bound = std::min<uint64_t>(g.K, n);
    const bool slotted = bound < g.K;
    const uint64_t pool_words = bound * 1024u;
    const OutLayout L = plan_out(bound, g.K, pool_words, 0, 0);
    CR_RET(alloc_out(out, L, bound, g.K, pool_words, 0, 0, s));
    out->max_key = max_key32;

    {
        CR_TIMED("ids_tile_sort", s);
        ids_tile_sort<false><<<g.G, TS_NT, 0, s>>>(d_ids, g, part, tab, gmax, tot, nullptr, wg_count);
    }
    CR_LAUNCH_CHECK();
    if (slotted) {
        uint32_t* pres = sc.at<uint32_t>(o_pres);
        CR_RET(fill_u32(pres, 0u, 2048u, s));
        {
            CR_TIMED("ids_presence", s);
            ids_presence<<<std::max(1u, std::min<uint32_t>((n + 255u) / 256u, 1024u)), 256, 0, s>>>(d_ids, n, g.K, pres);
        }
        CR_LAUNCH_CHECK();
        {
            CR_TIMED("ids_slots", s);
            ids_slots<<<1, 1024, 0, s>>>(pres, g.K, out->key_index);
        }
        CR_LAUNCH_CHECK();
    }
    HostSlotGuard hs;
    CR_RET(hs.acquire());
    {
        CR_TIMED("ids_build", s);
        const BuildMeta bm = bound >= g.K
                                 ? BuildMeta{out->keys, out->types, out->offsets, out->cardinalities, out->key_index}
                                 : BuildMeta{};
        ids_build<<<build_grid_persistent(g.NB, num_cus()), BUILD_NT, 0, s>>>(
            part, tab, g, wg_count, universe, false, slotted ? out->key_index : nullptr, out->bitmap_data, nullptr,
            key_count, tot, bm);
    }
    CR_LAUNCH_CHECK();
    {
        CR_TIMED("ids_rank", s);
        ids_rank<<<(g.K + 1023u) / 1024u, 1024, 0, s>>>(g, key_count, gmax, out->keys, out->types, out->offsets,
                                                         out->cardinalities, out->key_index, tot, hs.dev<IdsTotals>(),
                                                         slotted);
    }
    CR_LAUNCH_CHECK();
    CR_RET(sync_stream(s));
    IdsTotals h{};
    {
        const volatile IdsTotals* hp = hs.host<IdsTotals>();
        h.n_containers = hp->n_containers;
        h.err = hp->err;
        h.max_id = hp->max_id;
        h.moved = hp->moved;
        h.total = hp->total;
    }
    if (h.err) {
        free_async(out, s);
        set_error("upload_from_ids: an id's key exceeds max_key = (universe_size-1)>>16 = %u", max_key32);
        return CR_ERR_INVALID;
    }
    out->universe_size = universe;
    out->total_cardinality = h.total;
    out->n_containers = h.n_containers;
    out->n_bitmap_containers = h.n_containers;
    if (h.total <= static_cast<uint64_t>(universe) / 2u) {  // strict (:359)
        if (!h.moved) return CR_OK;
        // Present keys are not a prefix: a block of n_containers slots takes
        // the metadata and the containers in rank order.
        const uint64_t nc = h.n_containers;
        cr_gpu_roaring dense;
        reset(&dense);
        const OutLayout L3 = plan_out(nc, g.K, nc * 1024u, 0, 0);
        CR_RET(alloc_out(&dense, L3, nc, g.K, nc * 1024u, 0, 0, s));
        CopyList cl{};
        cl.seg[cl.n++] = {out->keys, dense.keys, nc * 2u};
        cl.seg[cl.n++] = {out->types, dense.types, nc};
        cl.seg[cl.n++] = {out->offsets, dense.offsets, nc * 4u};
        cl.seg[cl.n++] = {out->cardinalities, dense.cardinalities, nc * 2u};
        cl.seg[cl.n++] = {out->key_index, dense.key_index, static_cast<uint64_t>(g.K) * 2u};
        {
            CR_TIMED("ids_compact", s);
            CR_RET(copy_segments(cl, s));
            ids_gather_pool<<<static_cast<uint32_t>((nc + 3) / 4), 256, 0, s>>>(out->keys, static_cast<uint32_t>(nc),
                                                                                out->bitmap_data, dense.bitmap_data);
        }
        CR_LAUNCH_CHECK();
        dense.universe_size = universe;
        dense.max_key = max_key32;
        dense.total_cardinality = h.total;
        dense.n_containers = h.n_containers;
        dense.n_bitmap_containers = h.n_containers;
        free_async(out, s);
        *out = dense;
        return sync_stream(s);
    }
    if (h.total <= static_cast<uint64_t>(universe) / 2u) return CR_OK;  // strict (:359)

    // Complement path (:361-410): ids must lie in [0, U).
    if (h.max_id >= universe) {
        free_async(out, s);
        set_error("upload_from_ids: complement needs every id < universe_size (max id %u)", h.max_id);
        return CR_ERR_INVALID;
    }
    const uint64_t logical = h.total;
    cr_gpu_roaring comp;
    reset(&comp);
    const OutLayout L2 = plan_out(g.K, g.K, static_cast<uint64_t>(g.K) * 1024u, 0, 0);
    CR_RET(alloc_out(&comp, L2, g.K, g.K, static_cast<uint64_t>(g.K) * 1024u, 0, 0, s));
    {
        CR_TIMED("ids_keyscan_complement", s);
        ids_keyscan_complement<<<1, 1024, 0, s>>>(g, universe, key_count, comp.keys, comp.types, comp.offsets,
                                                  comp.key_index, tot);
    }
    CR_LAUNCH_CHECK();
    {
        CR_TIMED("ids_build", s);
        ids_build<<<build_grid_persistent(g.NB, num_cus()), BUILD_NT, 0, s>>>(
            part, tab, g, wg_count, universe, true, comp.key_index, comp.bitmap_data, comp.cardinalities, nullptr, tot,
            BuildMeta{});
    }
    CR_LAUNCH_CHECK();
    CR_RET(read_back(&h, tot, sizeof(h), s));
    free_async(out, s);
    *out = comp;
    out->universe_size = universe;
    out->max_key = max_key32;
    out->negated = true;
    out->total_cardinality = logical;  // logical count (:408)
    out->n_containers = h.n_containers;
    out->n_bitmap_containers = h.n_containers;
    if (h.n_containers == 0) {  // build_from_device_ids returns early on an empty set (:180-183)
        free_async(out, s);
        out->universe_size = universe;
        out->negated = true;
        out->total_cardinality = logical;
    }
    return CR_OK;
}

int upload_from_device_ids_impl(const uint32_t* d_ids, uint32_t n, uint32_t universe, uint32_t thr, hipStream_t s,
                                cr_gpu_roaring* out)
{
    reset(out);
    out->universe_size = universe;
    if (n == 0) return CR_OK;  // src/upload_ids.cu:578-582
    if (n > SMALL_MAX) return large_upload(d_ids, n, universe, s, out);
    const uint32_t eff = thr == CR_PROMOTE_AUTO ? resolve_auto_threshold(universe, -1) : thr;
    return small_upload(d_ids, n, universe, eff, s, out);
}

}  // namespace crimpl

using namespace crimpl;

extern "C" int cr_upload_from_device_ids(const uint32_t* d_ids, uint32_t n_ids, uint32_t universe_size,
                                         cr_stream_t stream, uint32_t bitmap_threshold, cr_gpu_roaring* out)
{
    if (!out || (n_ids && !d_ids)) {
        set_error("cr_upload_from_device_ids: invalid argument");
        return CR_ERR_INVALID;
    }
    reset(out);
    return produced(upload_from_device_ids_impl(d_ids, n_ids, universe_size, bitmap_threshold, as_stream(stream), out),
                    out, as_stream(stream));
}

extern "C" int cr_upload_from_ids(const uint32_t* ids, uint32_t n_ids, uint32_t universe_size, cr_stream_t stream,
                                  uint32_t bitmap_threshold, cr_gpu_roaring* out)
{
    if (!out || (n_ids && !ids)) {
        set_error("cr_upload_from_ids: invalid argument");
        return CR_ERR_INVALID;
    }
    hipStream_t s = as_stream(stream);
    reset(out);
    if (n_ids == 0) return produced(upload_from_device_ids_impl(nullptr, 0, universe_size, bitmap_threshold, s, out), out, s);
    Scratch sc;
    CR_RET(sc.alloc(static_cast<size_t>(n_ids) * 4u, s));
    CR_RET(h2d_pageable(sc.ptr, ids, static_cast<size_t>(n_ids) * 4u, s));
    return produced(upload_from_device_ids_impl(sc.at<uint32_t>(0), n_ids, universe_size, bitmap_threshold, s, out),
                    out, s);
}

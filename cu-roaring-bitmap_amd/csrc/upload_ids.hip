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

namespace crimpl {

constexpr uint32_t BK_SHIFT = 4;               // 16 keys per bucket
constexpr uint32_t BK_KEYS = 1u << BK_SHIFT;
constexpr uint32_t MAX_BUCKETS = 65536 / BK_KEYS;
constexpr int TS_NT = 1024;                    // tile-sort workgroup
constexpr uint32_t TS_PER = 24;                // ids per thread per tile
constexpr uint32_t TILE = TS_NT * TS_PER;      // 24576 ids: 96 KiB of LDS
// A sorted tile is stored as a bit stream of 20-bit fields, id & 0xFFFFF (the
// bucket is implied by the field's run): field i occupies bits [20 i, 20 i + 20)
// of the tile's slot of TILE_WORDS u32, 2.5 bytes an id.
constexpr uint32_t FIELD_BITS = 16 + BK_SHIFT;
constexpr uint32_t FIELD_MASK = (1u << FIELD_BITS) - 1u;
constexpr uint32_t TILE_WORDS = TILE * FIELD_BITS / 32;
static_assert(TILE_WORDS % 4 == 0, "tile slots hold whole 16-byte vectors");
static_assert(TILE <= 65535, "run starts are u16");
// Run table: tiles are grouped in blocks of TB; entry (block, bucket, slot) is
// the start of the bucket in tile block*TB + slot, so one bucket's starts for
// a block are TB contiguous u16 (the build reads a bucket's column).  The tile
// sort hands out whole blocks, so a block's rows fill up in one workgroup.
constexpr uint32_t TB = 8;
constexpr uint32_t STAGE_NB = 1024;  // run-table rows staged in LDS up to this many buckets

struct IdsTotals {
    uint32_t n_containers;
    uint32_t err;  // an id's key exceeded max_key
    uint32_t max_id;
    uint32_t moved;  // present keys are not a prefix: the pool needs compaction
    unsigned long long total;  // distinct ids (or complement count)
    uint32_t done;    // rank workgroups finished
    uint32_t absent;  // build workgroups that found a key of the universe with no id
};

struct IdsGeom {
    uint64_t n;
    uint32_t n_tiles;
    uint32_t G;   // tile-sort workgroups
    uint32_t K;   // keys in the universe (max_key + 1)
    uint32_t NB;  // buckets
    bool vec;     // ids pointer 16-byte aligned
};

// Each workgroup takes blocks of TB tiles.  A tile is counting-sorted by
// bucket in LDS and written back to its own slot of `part` (tile t at word
// t * TILE_WORDS) as packed fields, a streaming write; `tab` row t holds the
// tile's bucket starts (NB + 1 u16, in fields).  An id whose bucket lies past
// the universe's last goes to a sentinel bucket NB that is sorted after the
// others and neither written nor built; the error is raised from the maximum
// id, which each workgroup reports.  Every lane holds an id: a partial last
// tile is padded with ids of the sentinel bucket (which do not enter the
// maximum).
__global__ __launch_bounds__(TS_NT) void ids_tile_sort(const uint32_t* __restrict__ ids, IdsGeom g,
                                                       uint32_t* __restrict__ part, uint16_t* __restrict__ tab,
                                                       uint32_t* gmax, IdsTotals* tot)
{
    __shared__ uint32_t buf[TILE];
    __shared__ uint32_t cnt[MAX_BUCKETS + 1];
    // A block's run-table rows are staged here and written as one contiguous
    // copy when the block ends (up to STAGE_NB buckets; more write directly).
    __shared__ uint4 stage[STAGE_NB + 1];  // row i = TB u16 starts of bucket i
    __shared__ uint32_t lds[16];
    __shared__ uint32_t s_max;
    const uint32_t t = threadIdx.x;
    const uint32_t lane = __lane_id();
    const uint32_t NB = g.NB;
    const bool staged = NB <= STAGE_NB;
    if (t == 0) {
        s_max = 0;
        if (blockIdx.x == 0) {  // the build accumulates the distinct count
            tot->total = 0;
            tot->moved = 0;
            tot->n_containers = 0;  // the rank workgroups accumulate these
            tot->max_id = 0;
            tot->done = 0;
            tot->absent = 0;
        }
    }
    uint32_t mx = 0;
    // Returns whether the tile is partial; a partial tile's maximum is taken
    // here (over its real ids), a full tile's in the main loop, after the
    // prefetched loads have landed.
    auto load_ids = [&](uint32_t tl, uint32_t (&w)[TS_PER]) -> bool {
        const uint64_t base = static_cast<uint64_t>(tl) * TILE;
        const uint64_t hi = min(g.n, base + TILE);
        if (g.vec && hi - base == TILE) {
            const uint4* src = reinterpret_cast<const uint4*>(ids + base);
#pragma unroll
            for (uint32_t q = 0; q < TS_PER / 4; ++q) {
                const uint4 a = ld_stream(src + t + q * TS_NT);
                w[4 * q + 0] = a.x, w[4 * q + 1] = a.y, w[4 * q + 2] = a.z, w[4 * q + 3] = a.w;
            }
            return false;
        } else {
            const uint32_t* src = ids + base;  // wave-uniform base, 32-bit lane offsets
            const uint32_t rem = static_cast<uint32_t>(hi - base);
#pragma unroll
            for (uint32_t j = 0; j < TS_PER; ++j) {
                const uint32_t i = t + j * TS_NT;
                if (i < rem) {
                    w[j] = src[i];
                    if (rem < TILE) mx = max(mx, w[j]);
                } else {
                    // Padding of a partial last tile: 0xFFFFFFFF falls in the
                    // sentinel bucket; with 65536 keys there is none, and the
                    // pads repeat the tile's own ids, spread like the tile.
                    w[j] = NB < MAX_BUCKETS ? 0xFFFFFFFFu : src[i % rem];
                }
            }
            return rem < TILE;
        }
    };
    // The next tile's ids: the first half is loaded while the current tile is
    // scanned and scattered (into registers of its own), the second half once
    // the current tile's ids are in LDS, while it is packed and written.  (All
    // of it early would hold 48 ids a lane with the ranks, which spills, and a
    // spill reload waits for every outstanding load.)
    uint32_t v[TS_PER];
    bool partial = false;
    // Workgroup g takes blocks g, g + G, ...; `next` steps through them.
    auto next = [&](uint32_t tl) { return (tl % TB != TB - 1) ? tl + 1 : tl + 1 + (g.G - 1) * TB; };
    auto bucket = [&](uint32_t x) { return min(x >> (16 + BK_SHIFT), NB); };
    const uint32_t first = blockIdx.x * TB;
    if (first < g.n_tiles) partial = load_ids(first, v);
    for (uint32_t tile = first; tile < g.n_tiles; tile = next(tile)) {
        for (uint32_t i = t; i <= NB; i += TS_NT) cnt[i] = 0;
        __syncthreads();
        if (!partial) {
#pragma unroll
            for (uint32_t j = 0; j < TS_PER; ++j) mx = max(mx, v[j]);
        }
        // Ranks within the tile.  When every id of the wave's pass falls in
        // one bucket (clustered ids), a single atomic reserves them all.
        uint32_t rk[TS_PER / 2];  // tile ranks (< 24576) packed two per register
        const uint32_t b00 = __builtin_amdgcn_readfirstlane(bucket(v[0]));
        bool diff = false;
#pragma unroll
        for (uint32_t j = 0; j < TS_PER; ++j) diff |= bucket(v[j]) != b00;
        if (__ballot(diff) == 0) {
            uint32_t r0 = 0;
            if (lane == 0) r0 = atomicAdd(&cnt[b00], 64u * TS_PER);
            const uint32_t run = __builtin_amdgcn_readfirstlane(r0) + lane;
#pragma unroll
            for (uint32_t j = 0; j < TS_PER; j += 2) rk[j >> 1] = (run + 64u * j) | ((run + 64u * (j + 1)) << 16);
        } else {
#pragma unroll
            for (uint32_t j = 0; j < TS_PER; ++j) {
                const uint32_t r = atomicAdd(&cnt[bucket(v[j])], 1u);
                if (j & 1u)
                    rk[j >> 1] |= r << 16;
                else
                    rk[j >> 1] = r;
            }
        }
        // First half of the next tile's ids, when it is a whole aligned tile
        // (a partial or unaligned one is loaded late, by load_ids).
        const uint32_t nt = next(tile);
        const bool nfull = nt < g.n_tiles && g.vec && static_cast<uint64_t>(nt + 1) * TILE <= g.n;
        uint32_t vh[TS_PER / 2];
        if (nfull) {
            const uint4* src = reinterpret_cast<const uint4*>(ids + static_cast<uint64_t>(nt) * TILE);
#pragma unroll
            for (uint32_t q = 0; q < TS_PER / 8; ++q) {
                const uint4 a = ld_stream(src + t + q * TS_NT);
                vh[4 * q + 0] = a.x, vh[4 * q + 1] = a.y, vh[4 * q + 2] = a.z, vh[4 * q + 3] = a.w;
            }
        }
        __syncthreads();
        constexpr uint32_t BPT = MAX_BUCKETS / TS_NT;  // buckets scanned per thread
        uint32_t cv[BPT], cs = 0;
#pragma unroll
        for (uint32_t q = 0; q < BPT; ++q) {
            const uint32_t bq = t * BPT + q;
            cv[q] = bq < NB ? cnt[bq] : 0u;
            cs += cv[q];
        }
        uint32_t total;  // ids of the real buckets; the sentinel's follow
        uint32_t st = block_excl_scan<TS_NT>(cs, lds, total);
        // Bases, and the tile's column of the run table.
        uint16_t* trow_col = staged ? reinterpret_cast<uint16_t*>(stage) + tile % TB
                                    : tab + static_cast<uint64_t>(tile / TB) * (NB + 1) * TB + tile % TB;
#pragma unroll
        for (uint32_t q = 0; q < BPT; ++q) {
            const uint32_t bq = t * BPT + q;
            if (bq < NB) {
                cnt[bq] = st;
                trow_col[static_cast<uint64_t>(bq) * TB] = static_cast<uint16_t>(st);
            }
            st += cv[q];
        }
        if (t == 0) {
            cnt[NB] = total;
            trow_col[static_cast<uint64_t>(NB) * TB] = static_cast<uint16_t>(total);
        }
        __syncthreads();
#pragma unroll
        for (uint32_t j = 0; j < TS_PER; ++j) {
            uint32_t x = v[j];
            // An empty asm hides x's origin, so the bucket address is computed
            // again here instead of being kept in registers since the ranking.
            asm volatile("" : "+v"(x));
            buf[cnt[bucket(x)] + ((rk[j >> 1] >> ((j & 1u) * 16)) & 0xFFFFu)] = x;
        }
        __syncthreads();
        if (nfull) {
            const uint4* src = reinterpret_cast<const uint4*>(ids + static_cast<uint64_t>(nt) * TILE);
#pragma unroll
            for (uint32_t q = TS_PER / 8; q < TS_PER / 4; ++q) {
                const uint4 a = ld_stream(src + t + q * TS_NT);
                v[4 * q + 0] = a.x, v[4 * q + 1] = a.y, v[4 * q + 2] = a.z, v[4 * q + 3] = a.w;
            }
#pragma unroll
            for (uint32_t j = 0; j < TS_PER / 2; ++j) v[j] = vh[j];
            partial = false;
        } else if (nt < g.n_tiles) {
            partial = load_ids(nt, v);
        }
        if (staged && (tile % TB == TB - 1 || tile + 1 == g.n_tiles)) {  // the block's rows, contiguous
            uint4* trow = reinterpret_cast<uint4*>(tab + static_cast<uint64_t>(tile / TB) * (NB + 1) * TB);
            for (uint32_t i = t; i <= NB; i += TS_NT) trow[i] = stage[i];
        }
        // Packing in place: thread g turns fields [8 g, 8 g + 8) (two 16-byte
        // LDS reads) into words [5 g, 5 g + 5) of the stream, which overwrite
        // the tile's front after a barrier; then the 16-byte vectors holding
        // real buckets' fields stream out.
        static_assert(FIELD_BITS == 20 && TILE % (8 * TS_NT) == 0, "8 fields -> 5 words, whole passes");
        constexpr uint32_t GPT = TILE / (8 * TS_NT);  // 8-field groups per thread
        uint32_t pw[GPT][5];
#pragma unroll
        for (uint32_t k = 0; k < GPT; ++k) {
            const uint4* src = reinterpret_cast<const uint4*>(buf) + 2u * (t + k * TS_NT);
            const uint4 a = src[0], c = src[1];
            const uint32_t f0 = a.x & FIELD_MASK, f1 = a.y & FIELD_MASK, f2 = a.z & FIELD_MASK, f3 = a.w & FIELD_MASK;
            const uint32_t f4 = c.x & FIELD_MASK, f5 = c.y & FIELD_MASK, f6 = c.z & FIELD_MASK, f7 = c.w & FIELD_MASK;
            pw[k][0] = f0 | (f1 << 20);
            pw[k][1] = (f1 >> 12) | (f2 << 8) | (f3 << 28);
            pw[k][2] = (f3 >> 4) | (f4 << 16);
            pw[k][3] = (f4 >> 16) | (f5 << 4) | (f6 << 24);
            pw[k][4] = (f6 >> 8) | (f7 << 12);
        }
        __syncthreads();
#pragma unroll
        for (uint32_t k = 0; k < GPT; ++k)
#pragma unroll
            for (uint32_t q = 0; q < 5u; ++q) buf[5u * (t + k * TS_NT) + q] = pw[k][q];
        __syncthreads();
        uint4* dst = reinterpret_cast<uint4*>(part + static_cast<uint64_t>(tile) * TILE_WORDS);
        const uint32_t n4 = (FIELD_BITS * total + 127u) >> 7;
        for (uint32_t u = t; u < n4; u += TS_NT) st_stream(dst + u, reinterpret_cast<const uint4*>(buf)[u]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = max(mx, static_cast<uint32_t>(__shfl_xor(mx, o, 64)));
    if (lane == 0) atomicMax(&s_max, mx);
    __syncthreads();
    if (t == 0) gmax[blockIdx.x] = s_max;  // per-workgroup partials: nothing here needs zeroed memory
}

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
                                                 uint16_t* key_index, IdsTotals* tot, IdsTotals* host)
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
        moved = rank != k;
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

// One workgroup per bucket: its 16 containers as 16 x 2048 u32 LDS words
// (128 KiB), filled from the bucket's run in every tile (the bucket order over
// the XCDs is below).
// Normal mode writes each present key's container to pool slot `key`, every
// key's distinct count, and the metadata as if ranks were keys (right when
// every key is present; ids_rank rewrites it otherwise, told by `absent`);
// complement mode writes ~bits masked to [0, U) at the key_index rank of keys
// whose complement is non-empty, with their cards.
constexpr int BUILD_NT = 1024;
constexpr uint32_t BUILD_WAVES = BUILD_NT / 64;

// Workgroups go round-robin over the 8 XCDs; XCD x takes the contiguous
// bucket range [x * per, (x + 1) * per), in order, so almost every pair of
// neighbouring buckets -- whose runs share the cache line at their boundary in
// every tile -- runs on one XCD, close in time, and that line comes from its L2.
__host__ __device__ inline uint32_t build_per_xcd(uint32_t nb) { return (nb + 7) / 8; }
inline uint32_t build_grid(uint32_t nb) { return 8 * build_per_xcd(nb); }

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

__global__ __launch_bounds__(BUILD_NT) void ids_build(const uint32_t* __restrict__ part,
                                                      const uint16_t* __restrict__ tab, IdsGeom g, uint32_t universe,
                                                      bool complement, const uint16_t* key_index,
                                                      uint64_t* __restrict__ pool, uint16_t* cards,
                                                      uint32_t* key_count, IdsTotals* tot, BuildMeta m)
{
    __shared__ alignas(16) uint32_t bits[BK_KEYS * 2048u];  // 128 KiB of the CU's 160 KiB LDS
    const uint32_t t = threadIdx.x;
    const uint32_t b = (blockIdx.x % 8) * build_per_xcd(g.NB) + blockIdx.x / 8;
    if (b >= g.NB) return;
    for (uint32_t i = t; i < BK_KEYS * 512u; i += BUILD_NT) reinterpret_cast<uint4*>(bits)[i] = make_uint4(0, 0, 0, 0);
    __syncthreads();
    const uint32_t wave = t >> 6;
    const uint32_t lane = __lane_id();
    const uint32_t grp = lane >> 2;  // sixteen 4-lane groups
    const uint32_t r4 = lane & 3u;
    const uint32_t n_blk = (g.n_tiles + TB - 1) / TB;
    // Wave w owns tile blocks w, w + 16, ...; a step covers 64 / TB of them
    // (one tile per lane, its run bounds loaded a step ahead: the TB lanes of
    // a block read TB contiguous u16).  Each 4-lane group reads four tiles'
    // runs as 16-word windows (64 bytes, 25.6 fields) with 16-byte loads
    // aligned down to 4 words, and the loads of the first two windows are all
    // issued before any bit is set.  A lane takes the fields that start in its
    // 4 words; one that ends past them takes its last bits from the next
    // word: the next lane's first, or for the group's last lane one more load.
    constexpr uint32_t BPS = 64u / TB;  // blocks per step
    const uint32_t per_wave = n_blk > wave ? (n_blk - wave + BUILD_WAVES - 1) / BUILD_WAVES : 0u;
    auto tile_of = [&](uint32_t st, uint32_t l) { return (wave + BUILD_WAVES * (st * BPS + l / TB)) * TB + l % TB; };
    auto tab_load = [&](uint32_t st, uint32_t& r0, uint32_t& r1) {
        r0 = r1 = 0;
        const uint32_t jb = st * BPS + lane / TB;
        const uint32_t tile = tile_of(st, lane);
        if (jb < per_wave && tile < g.n_tiles) {
            const uint16_t* tc =
                tab + (static_cast<uint64_t>(wave + BUILD_WAVES * jb) * (g.NB + 1) + b) * TB + lane % TB;
            r0 = tc[0];
            r1 = tc[TB];
        }
    };
    // Fields of [s0, s1) starting in words lo_w .. lo_w + 3 (x), with c4 =
    // word lo_w + 4.  The first starts o < 20 bits in; after a funnel shift by
    // o, field m sits at bit 20 m (m = 6 only when o < 8).
    auto set_chunk = [&](const uint4& x, uint32_t c4, uint32_t lo_w, uint32_t s0, uint32_t s1) {
        static_assert(FIELD_BITS == 20, "the unpacking below assumes 20-bit fields");
        const uint32_t C = 32u * lo_w;
        const uint32_t i0 = (C + FIELD_BITS - 1u) / FIELD_BITS;
        const uint32_t o = FIELD_BITS * i0 - C;
        const uint32_t d0 = __builtin_amdgcn_alignbit(x.y, x.x, o);
        const uint32_t d1 = __builtin_amdgcn_alignbit(x.z, x.y, o);
        const uint32_t d2 = __builtin_amdgcn_alignbit(x.w, x.z, o);
        const uint32_t d3 = __builtin_amdgcn_alignbit(c4, x.w, o);
        const uint32_t d4 = c4 >> o;
        const uint32_t f[7] = {d0,
                               __builtin_amdgcn_alignbit(d1, d0, 20),
                               d1 >> 8,
                               __builtin_amdgcn_alignbit(d2, d1, 28),
                               __builtin_amdgcn_alignbit(d3, d2, 16),
                               d3 >> 4,
                               __builtin_amdgcn_alignbit(d4, d3, 24)};
#pragma unroll
        for (uint32_t m = 0; m < 7u; ++m) {
            const uint32_t i = i0 + m;
            if (i >= s0 && i < s1 && (m < 6u || o < 8u)) {
                const uint32_t F = f[m] & FIELD_MASK;  // key-in-bucket << 16 | low 16 bits
                atomicOr(&bits[F >> 5], 1u << (F & 31u));
            }
        }
    };
    uint32_t n0, n1;
    tab_load(0, n0, n1);
    for (uint32_t st = 0; st * BPS < per_wave; ++st) {
        const uint32_t m0 = n0, m1 = n1;
        tab_load(st + 1, n0, n1);
        // windows from the 16-byte-aligned word holding field m0 to the last
        // word holding the run's bits
        uint32_t nw = m1 > m0 ? (((FIELD_BITS * m1 - 1u) >> 5) - (((FIELD_BITS * m0) >> 5) & ~3u)) / 16u + 1u : 0u;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) nw = max(nw, static_cast<uint32_t>(__shfl_xor(nw, o, 64)));
        uint32_t ts0[4], ts1[4], tb[4], wb[4], we[4];
#pragma unroll
        for (uint32_t h = 0; h < 4u; ++h) {
            const uint32_t src = 16u * h + grp;
            ts0[h] = __shfl(m0, static_cast<int>(src), 64);
            ts1[h] = __shfl(m1, static_cast<int>(src), 64);
            tb[h] = tile_of(st, src) * TILE_WORDS;  // < 2^32 words for n < 2^32 (past the end: empty runs)
            wb[h] = ((FIELD_BITS * ts0[h]) >> 5) & ~3u;
            we[h] = ts1[h] > ts0[h] ? (FIELD_BITS * ts1[h] - 1u) >> 5 : 0u;
        }
        // A lane loads when its first word holds run bits (lo_w <= we, so its
        // 4 words stay in the tile's written vectors); the last lane's extra
        // word only when the run reaches it.
        auto window = [&](uint32_t h, uint32_t k, uint4& x, uint32_t& e) {
            const uint32_t lo_w = wb[h] + 16u * k + 4u * r4;
            const bool act = ts1[h] > ts0[h] && lo_w <= we[h];
            x = act ? *reinterpret_cast<const uint4*>(part + tb[h] + lo_w) : make_uint4(0, 0, 0, 0);
            e = (act && r4 == 3u && lo_w + 4u <= we[h]) ? part[tb[h] + lo_w + 4u] : 0u;
        };
        {
            uint4 x[4][2];
            uint32_t e[4][2];
#pragma unroll
            for (uint32_t h = 0; h < 4u; ++h)
#pragma unroll
                for (uint32_t k = 0; k < 2u; ++k) window(h, k, x[h][k], e[h][k]);
#pragma unroll
            for (uint32_t h = 0; h < 4u; ++h)
#pragma unroll
                for (uint32_t k = 0; k < 2u; ++k) {
                    const uint32_t nx = __shfl_down(x[h][k].x, 1, 64);
                    set_chunk(x[h][k], r4 == 3u ? e[h][k] : nx, wb[h] + 16u * k + 4u * r4, ts0[h], ts1[h]);
                }
        }
        for (uint32_t k = 2; k < nw; ++k) {  // runs longer than two windows (clustered ids)
#pragma unroll
            for (uint32_t h = 0; h < 4u; ++h) {
                uint4 x;
                uint32_t e;
                window(h, k, x, e);
                const uint32_t nx = __shfl_down(x.x, 1, 64);
                set_chunk(x, r4 == 3u ? e : nx, wb[h] + 16u * k + 4u * r4, ts0[h], ts1[h]);
            }
        }
    }
    __syncthreads();
    __shared__ uint32_t wave_pc[BUILD_WAVES];
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
                uint32_t x[4] = {~v[q].x, ~v[q].y, ~v[q].z, ~v[q].w};
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (i0 + e >= valid_words) x[e] = (i0 + e == valid_words) ? (x[e] & tail_mask) : 0u;
                v[q] = make_uint4(x[0], x[1], x[2], x[3]);
            }
            pc += __popc(v[q].x) + __popc(v[q].y) + __popc(v[q].z) + __popc(v[q].w);
        }
        pc = wave_sum(pc);
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
            const uint32_t slot = complement ? key_index[key] : key;
            uint4* dst = reinterpret_cast<uint4*>(pool + static_cast<uint64_t>(slot) * 1024u);
#pragma unroll
            for (int q = 0; q < 8; ++q) st_stream(dst + lane + 64 * q, v[q]);
            if (complement && lane == 0) cards[slot] = static_cast<uint16_t>(pc > 65535u ? 0u : pc);
        }
    }
    if (lane == 0) wave_pc[c] = pc;
    __syncthreads();
    if (t == 0) {  // device atomics without a return, so the workgroup retires at once
        unsigned long long s = 0;
        bool absent = false;
        for (uint32_t i = 0; i < BUILD_WAVES; ++i) {
            s += wave_pc[i];
            absent |= b * BK_KEYS + i < g.K && wave_pc[i] == 0;
        }
        if (s) atomicAdd(&tot->total, s);
        if (!complement && absent) atomicAdd(&tot->absent, 1u);
    }
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
__global__ __launch_bounds__(1024) void ids_small_write(const SmallPlan* plan, uint32_t thr, uint16_t* keys,
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
    const uint64_t bmp_words = static_cast<uint64_t>(plan->n_bitmap) * 1024u;
    for (uint64_t i = t; i < bmp_words; i += 1024) bmp[i] = 0;
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
        } else {
            types[c] = CR_ARRAY;
            offsets[c] = s_aoff[c] * 2u;
            for (uint32_t i = s; i < e; ++i) arr[s_aoff[c] + (i - s)] = static_cast<uint16_t>(plan->vals[i]);
        }
    }
    __syncthreads();
    // bitmap bits: one lane per value (atomicOr: values of one container share words)
    for (uint32_t c = 0; c < nc; ++c) {
        const uint32_t s = plan->cstart[c], e = plan->cstart[c + 1];
        if (e - s <= thr) continue;
        uint64_t* dst = bmp + static_cast<uint64_t>(s_bslot[c]) * 1024u;
        for (uint32_t i = s + t; i < e; i += 1024) {
            const uint32_t low = plan->vals[i] & 0xFFFFu;
            atomicOr(reinterpret_cast<unsigned long long*>(&dst[low >> 6]), 1ull << (low & 63u));
        }
    }
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
    CR_RET(sync_stream(s));
    return CR_OK;
}

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
    const size_t o_part = c.add(sizeof(uint32_t) * (static_cast<uint64_t>(g.n_tiles) * TILE_WORDS + 4));
    Scratch sc;
    CR_RET(sc.alloc(c.total, s));
    uint32_t* gmax = sc.at<uint32_t>(o_gmax);
    uint32_t* key_count = sc.at<uint32_t>(o_kc);
    IdsTotals* tot = sc.at<IdsTotals>(o_tot);
    uint16_t* tab = sc.at<uint16_t>(o_tab);
    uint32_t* part = sc.at<uint32_t>(o_part);

    // Containers <= min(keys, ids) bounds the metadata; the pool is addressed
    // by key (slot k holds key k's container) until the ranks are known.
    const uint64_t bound = std::min<uint64_t>(g.K, n);
    const uint64_t pool_words = static_cast<uint64_t>(g.K) * 1024u;
    const OutLayout L = plan_out(bound, g.K, pool_words, 0, 0);
    CR_RET(alloc_out(out, L, bound, g.K, pool_words, 0, 0, s));
    out->max_key = max_key32;

    {
        CR_TIMED("ids_tile_sort", s);
        ids_tile_sort<<<g.G, TS_NT, 0, s>>>(d_ids, g, part, tab, gmax, tot);
    }
    CR_LAUNCH_CHECK();
    HostSlotGuard hs;
    CR_RET(hs.acquire());
    {
        CR_TIMED("ids_build", s);
        const BuildMeta bm = bound >= g.K
                                 ? BuildMeta{out->keys, out->types, out->offsets, out->cardinalities, out->key_index}
                                 : BuildMeta{};
        ids_build<<<build_grid(g.NB), BUILD_NT, 0, s>>>(part, tab, g, universe, false, nullptr, out->bitmap_data,
                                                        nullptr, key_count, tot, bm);
    }
    CR_LAUNCH_CHECK();
    {
        CR_TIMED("ids_rank", s);
        ids_rank<<<(g.K + 1023u) / 1024u, 1024, 0, s>>>(g, key_count, gmax, out->keys, out->types, out->offsets,
                                                         out->cardinalities, out->key_index, tot, hs.dev<IdsTotals>());
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
        ids_build<<<build_grid(g.NB), BUILD_NT, 0, s>>>(part, tab, g, universe, true, comp.key_index,
                                                    comp.bitmap_data, comp.cardinalities, nullptr, tot, BuildMeta{});
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
    return upload_from_device_ids_impl(d_ids, n_ids, universe_size, bitmap_threshold, as_stream(stream), out);
}

extern "C" int cr_upload_from_ids(const uint32_t* ids, uint32_t n_ids, uint32_t universe_size, cr_stream_t stream,
                                  uint32_t bitmap_threshold, cr_gpu_roaring* out)
{
    if (!out || (n_ids && !ids)) {
        set_error("cr_upload_from_ids: invalid argument");
        return CR_ERR_INVALID;
    }
    hipStream_t s = as_stream(stream);
    if (n_ids == 0) return upload_from_device_ids_impl(nullptr, 0, universe_size, bitmap_threshold, s, out);
    Scratch sc;
    CR_RET(sc.alloc(static_cast<size_t>(n_ids) * 4u, s));
    CR_RET(h2d_pageable(sc.ptr, ids, static_cast<size_t>(n_ids) * 4u, s));
    return upload_from_device_ids_impl(sc.at<uint32_t>(0), n_ids, universe_size, bitmap_threshold, s, out);
}

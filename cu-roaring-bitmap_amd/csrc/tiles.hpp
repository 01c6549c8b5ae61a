// The tile sort of ids (or query ids) by 16-key bucket and the walk over one
// bucket's runs, shared by upload_from_ids (which sets each id's bit in the
// bucket's LDS containers) and the partitioned point queries (which test it).
//
// Ids are grouped by 16-key bucket (1 MiB of id space) inside 24576-id tiles:
// each tile is counting-sorted by bucket in LDS and streamed back to its own
// slot as 20-bit fields (the id within its bucket), with the tile's bucket
// starts in a small table.  A bucket's consumer -- one workgroup holding the
// bucket's 16 containers in 128 KiB of LDS -- then reads the bucket's run in
// every tile (~24 fields, 60 bytes, at 2^30).
#pragma once
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
// maximum).  With PERM, perm[t * TILE + p] receives the padded sorted position
// (within tile t) of the tile's p-th id, padding ids included: rank r in
// bucket b, whose run starts at sorted position S, gets ((S + 7 b + 7) & ~7) + r,
// so every bucket's positions start at a multiple of 8 and no two buckets'
// positions share a group of 8.
template <bool PERM>
__global__ __launch_bounds__(TS_NT) void ids_tile_sort(const uint32_t* __restrict__ ids, IdsGeom g,
                                                       uint32_t* __restrict__ part, uint16_t* __restrict__ tab,
                                                       uint32_t* gmax, IdsTotals* tot, uint16_t* __restrict__ perm)
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
    bool tile_vec = false;  // the current tile came in through 16-byte loads (id order 4 (t + q TS_NT) + r)
    // Workgroup g takes blocks g, g + G, ...; `next` steps through them.
    auto next = [&](uint32_t tl) { return (tl % TB != TB - 1) ? tl + 1 : tl + 1 + (g.G - 1) * TB; };
    auto bucket = [&](uint32_t x) { return min(x >> (16 + BK_SHIFT), NB); };
    const uint32_t first = blockIdx.x * TB;
    auto whole_vec = [&](uint32_t tl) { return g.vec && static_cast<uint64_t>(tl + 1) * TILE <= g.n; };
    if (first < g.n_tiles) {
        partial = load_ids(first, v);
        tile_vec = whole_vec(first);
    }
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
            // Per pass j, likewise when the wave's j-th ids share a bucket
            // (sorted or clustered ids spread over a few buckets per tile);
            // otherwise an atomic a lane.
#pragma unroll
            for (uint32_t j = 0; j < TS_PER; ++j) {
                const uint32_t bj = bucket(v[j]);
                const uint32_t b0 = __builtin_amdgcn_readfirstlane(bj);
                uint32_t r;
                if (__ballot(bj != b0) == 0) {
                    uint32_t r0 = 0;
                    if (lane == 0) r0 = atomicAdd(&cnt[b0], 64u);
                    r = __builtin_amdgcn_readfirstlane(r0) + lane;
                } else {
                    r = atomicAdd(&cnt[bj], 1u);
                }
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
                // with PERM the padded start rides in the high half
                cnt[bq] = PERM ? st | (((st + 7u * bq + 7u) & ~7u) << 16) : st;
                trow_col[static_cast<uint64_t>(bq) * TB] = static_cast<uint16_t>(st);
            }
            st += cv[q];
        }
        if (t == 0) {
            cnt[NB] = PERM ? total | (((total + 7u * NB + 7u) & ~7u) << 16) : total;
            trow_col[static_cast<uint64_t>(NB) * TB] = static_cast<uint16_t>(total);
        }
        __syncthreads();
#pragma unroll
        for (uint32_t j = 0; j < TS_PER; ++j) {
            uint32_t x = v[j];
            // An empty asm hides x's origin, so the bucket address is computed
            // again here instead of being kept in registers since the ranking.
            asm volatile("" : "+v"(x));
            const uint32_t c = cnt[bucket(x)];
            const uint32_t r = (rk[j >> 1] >> ((j & 1u) * 16)) & 0xFFFFu;
            buf[(PERM ? c & 0xFFFFu : c) + r] = x;
            if constexpr (PERM) {
                // the rank's half of rk now holds the padded sorted position:
                // bucket b's run starts at (start + 7 b) rounded up to a
                // multiple of 8, so each bucket's answers fill whole bytes
                // (< 24576 + 7 * 4096 + 7, fits 16 bits)
                const uint32_t pp = (c >> 16) + r;
                rk[j >> 1] = (j & 1u) ? ((rk[j >> 1] & 0xFFFFu) | (pp << 16)) : ((rk[j >> 1] & 0xFFFF0000u) | pp);
            }
        }
        if constexpr (PERM) {  // the ids' sorted positions, in the order load_ids placed them
            uint16_t* pt = perm + static_cast<uint64_t>(tile) * TILE;
            if (tile_vec) {  // id j = 4 q + r sits at 4 (t + q TS_NT) + r: one 8-byte store per q
#pragma unroll
                for (uint32_t q = 0; q < TS_PER / 4; ++q)
                    reinterpret_cast<uint2*>(pt)[t + q * TS_NT] = make_uint2(rk[2 * q], rk[2 * q + 1]);
            } else {  // id j sits at t + j TS_NT
#pragma unroll
                for (uint32_t j = 0; j < TS_PER; ++j)
                    pt[t + j * TS_NT] = static_cast<uint16_t>((rk[j >> 1] >> ((j & 1u) * 16)) & 0xFFFFu);
            }
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
            tile_vec = true;
        } else if (nt < g.n_tiles) {
            partial = load_ids(nt, v);
            tile_vec = whole_vec(nt);
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

constexpr int BUILD_NT = 1024;
constexpr uint32_t BUILD_WAVES = BUILD_NT / 64;

// Workgroups go round-robin over the 8 XCDs; XCD x takes the contiguous
// bucket range [x * per, (x + 1) * per), in order, so almost every pair of
// neighbouring buckets -- whose runs share the cache line at their boundary in
// every tile -- runs on one XCD, close in time, and that line comes from its L2.
__host__ __device__ inline uint32_t build_per_xcd(uint32_t nb) { return (nb + 7) / 8; }
inline uint32_t build_grid(uint32_t nb) { return 8 * build_per_xcd(nb); }

// Calls on_field(tile, i, F) for every field of bucket b's run in every tile:
// field i of tile `tile`'s sorted order, F = the id's low FIELD_BITS bits
// (key-in-bucket << 16 | low 16 bits).  Every thread of the BUILD_NT-thread
// workgroup calls it (wave = t >> 6, lane = its lane); fields arrive in no
// particular order and each exactly once.
// Runs longer than WALK_LONG windows (sorted or clustered ids) are queued in
// LDS and their remaining windows shared by the whole workgroup after the
// walk, so that a bucket whose ids sit in a few tiles -- one wave's blocks --
// keeps all sixteen waves busy (a run that finds the queue full is finished by
// its own wave); shorter runs stay with their own groups.  Every thread of the
// workgroup must call this.
constexpr uint32_t WALK_QCAP = 2048;  // 16 KiB of LDS beside the callers' 128 KiB
constexpr uint32_t WALK_LONG = 16;    // windows above which a run is queued (one window a group)

template <class OnField>
__device__ __forceinline__ void walk_bucket(const uint32_t* __restrict__ part, const uint16_t* __restrict__ tab,
                                            const IdsGeom& g, uint32_t b, uint32_t wave, uint32_t lane,
                                            OnField on_field)
{
    __shared__ uint2 q_ent[WALK_QCAP];  // {tile, s0 | s1 << 16}
    __shared__ uint32_t q_n;
    if (threadIdx.x == 0) q_n = 0;
    __syncthreads();
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
    auto set_chunk = [&](const uint4& x, uint32_t c4, uint32_t lo_w, uint32_t s0, uint32_t s1, uint32_t tile) {
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
            if (i >= s0 && i < s1 && (m < 6u || o < 8u)) on_field(tile, i, f[m] & FIELD_MASK);
        }
    };
    uint32_t n0, n1;
    tab_load(0, n0, n1);
    for (uint32_t st = 0; st * BPS < per_wave; ++st) {
        const uint32_t m0 = n0, m1 = n1;
        tab_load(st + 1, n0, n1);
        // windows from the 16-byte-aligned word holding field m0 to the last
        // word holding the run's bits
        const uint32_t own_nw =
            m1 > m0 ? (((FIELD_BITS * m1 - 1u) >> 5) - (((FIELD_BITS * m0) >> 5) & ~3u)) / 16u + 1u : 0u;
        uint32_t ts0[4], ts1[4], tb[4], wb[4], we[4], tl[4];
#pragma unroll
        for (uint32_t h = 0; h < 4u; ++h) {
            const uint32_t src = 16u * h + grp;
            ts0[h] = __shfl(m0, static_cast<int>(src), 64);
            ts1[h] = __shfl(m1, static_cast<int>(src), 64);
            tl[h] = tile_of(st, src);
            tb[h] = tl[h] * TILE_WORDS;  // < 2^32 words for n < 2^32 (past the end: empty runs)
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
                    set_chunk(x[h][k], r4 == 3u ? e[h][k] : nx, wb[h] + 16u * k + 4u * r4, ts0[h], ts1[h], tl[h]);
                }
        }
        // Runs of 3 .. WALK_LONG windows: the rest of their windows by their
        // own groups, all of the wave's runs together (the loop runs to the
        // wave's longest such run).
        uint32_t nw_mid = own_nw <= WALK_LONG ? own_nw : 0u;
#pragma unroll
        for (int d = 32; d > 0; d >>= 1) nw_mid = max(nw_mid, static_cast<uint32_t>(__shfl_xor(nw_mid, d, 64)));
        bool mid[4];
#pragma unroll
        for (uint32_t h = 0; h < 4u; ++h)
            mid[h] = static_cast<uint32_t>(__shfl(own_nw, static_cast<int>(16u * h + grp), 64)) <= WALK_LONG;
        for (uint32_t k = 2; k < nw_mid; ++k) {
#pragma unroll
            for (uint32_t h = 0; h < 4u; ++h) {
                uint4 x = make_uint4(0, 0, 0, 0);
                uint32_t e = 0;
                if (mid[h]) window(h, k, x, e);
                const uint32_t nx = __shfl_down(x.x, 1, 64);
                if (mid[h]) set_chunk(x, r4 == 3u ? e : nx, wb[h] + 16u * k + 4u * r4, ts0[h], ts1[h], tl[h]);
            }
        }
        // Longer runs: queued for the workgroup; one that finds the queue full
        // is finished here, one tile at a time, its remaining windows shared
        // by the wave's sixteen groups.
        const bool is_long = own_nw > WALK_LONG;
        uint32_t slot = WALK_QCAP;
        if (is_long) slot = atomicAdd(&q_n, 1u);
        if (is_long && slot < WALK_QCAP) q_ent[slot] = make_uint2(tile_of(st, lane), m0 | (m1 << 16));
        uint64_t longs = __ballot(is_long && slot >= WALK_QCAP);
        while (longs) {
            const uint32_t src = static_cast<uint32_t>(__builtin_ctzll(longs));
            longs &= longs - 1u;
            const uint32_t s0 = __shfl(m0, static_cast<int>(src), 64);
            const uint32_t s1 = __shfl(m1, static_cast<int>(src), 64);
            const uint32_t tile = tile_of(st, src);
            const uint32_t base = tile * TILE_WORDS;
            const uint32_t w0 = ((FIELD_BITS * s0) >> 5) & ~3u;
            const uint32_t w1 = (FIELD_BITS * s1 - 1u) >> 5;
            const uint32_t nwt = (w1 - w0) / 16u + 1u;
            for (uint32_t kb = 2; kb < nwt; kb += 16u) {  // wave-uniform trip count
                const uint32_t lo_w = w0 + 16u * (kb + grp) + 4u * r4;
                const bool act = lo_w <= w1;
                const uint4 x = act ? *reinterpret_cast<const uint4*>(part + base + lo_w) : make_uint4(0, 0, 0, 0);
                const uint32_t e = (act && r4 == 3u && lo_w + 4u <= w1) ? part[base + lo_w + 4u] : 0u;
                const uint32_t nx = __shfl_down(x.x, 1, 64);
                if (act) set_chunk(x, r4 == 3u ? e : nx, lo_w, s0, s1, tile);
            }
        }
    }
    // The queued runs: windows 2, 3, ... of each in chunks of sixteen (one a
    // group), the chunks of all runs dealt to the waves in turn.
    __syncthreads();
    const uint32_t nq = min(q_n, WALK_QCAP);
    uint32_t off = 0;  // chunks of the runs before
    for (uint32_t j = 0; j < nq; ++j) {
        const uint2 ent = q_ent[j];
        const uint32_t tile = ent.x, s0 = ent.y & 0xFFFFu, s1 = ent.y >> 16;
        const uint32_t base = tile * TILE_WORDS;
        const uint32_t w0 = ((FIELD_BITS * s0) >> 5) & ~3u;
        const uint32_t w1 = (FIELD_BITS * s1 - 1u) >> 5;
        const uint32_t nch = ((w1 - w0) / 16u - 1u + 15u) / 16u;  // windows 2 .. (w1 - w0) / 16
        for (uint32_t c = (wave + BUILD_WAVES - off % BUILD_WAVES) % BUILD_WAVES; c < nch; c += BUILD_WAVES) {
            const uint32_t lo_w = w0 + 16u * (2u + 16u * c + grp) + 4u * r4;
            const bool act = lo_w <= w1;
            const uint4 x = act ? *reinterpret_cast<const uint4*>(part + base + lo_w) : make_uint4(0, 0, 0, 0);
            const uint32_t e = (act && r4 == 3u && lo_w + 4u <= w1) ? part[base + lo_w + 4u] : 0u;
            const uint32_t nx = __shfl_down(x.x, 1, 64);
            if (act) set_chunk(x, r4 == 3u ? e : nx, lo_w, s0, s1, tile);
        }
        off += nch;
    }
}

}  // namespace crimpl

// The tile sort of ids (or query ids) by 16-key bucket and the walk over one
// bucket's runs, shared by upload_from_ids (which sets each id's bit in the
// bucket's LDS containers) and the partitioned point queries (which test it).
//
// Ids are grouped by 16-key bucket (1 MiB of id space) inside 24576-id tiles:
// each tile is counting-sorted by bucket in LDS and written back to its own
// slot as 20-bit fields (the id within its bucket), with the tile's bucket
// starts in a small table.  A bucket's consumer -- one workgroup holding the
// bucket's 16 containers in 128 KiB of LDS -- then reads the bucket's run in
// every tile (~24 fields, 60 bytes, at 2^30).
#pragma once
#include <type_traits>

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
constexpr uint32_t STAGE_W = STAGE_NB + 8;  // u16 per staged slot: buckets 0..STAGE_NB, 16-byte rows

struct IdsTotals {
    uint32_t n_containers;
    uint32_t err;  // an id's key exceeded max_key
    uint32_t max_id;
    uint32_t moved;  // present keys are not a prefix: the pool needs compaction
    unsigned long long total;  // distinct ids (or complement count)
    uint32_t done;    // rank workgroups finished
    uint32_t absent;  // build workgroups that found a key of the universe with no id
    uint32_t ticket[8];  // the build's next bucket (in its order) per XCD's range
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
// t * TILE_WORDS) as packed fields (ordinary stores, so that the tiles stay in
// the Infinity Cache for their reader); `tab` row t holds the
// tile's bucket starts (NB + 1 u16, in fields).  An id whose bucket lies past
// the universe's last goes to a sentinel bucket NB that is sorted after the
// others and neither written nor built; the error is raised from the maximum
// id, which each workgroup reports.  Every lane holds an id: a partial last
// tile is padded with ids of the sentinel bucket (which do not enter the
// maximum).  With PERM, perm[t * TILE + p] receives the padded sorted position
// (within tile t) of the tile's p-th id, padding ids included: rank r in
// bucket b, whose run starts at sorted position S, gets ((S + 7 b + 7) & ~7) + r,
// so every bucket's positions start at a multiple of 8 and no two buckets'
// positions share a group of 8.  With `wg_count` non-null, row w (NB u32)
// receives the number of ids workgroup w sorted into each real bucket, which
// the build sums into per-bucket totals to order its buckets.
template <bool PERM>
__global__ __launch_bounds__(TS_NT) void ids_tile_sort(const uint32_t* __restrict__ ids, IdsGeom g,
                                                       uint32_t* __restrict__ part, uint16_t* __restrict__ tab,
                                                       uint32_t* gmax, IdsTotals* tot, uint16_t* __restrict__ perm,
                                                       uint32_t* __restrict__ wg_count)
{
    __shared__ uint32_t buf[TILE];
    __shared__ alignas(16) uint32_t cnt[MAX_BUCKETS + 1];
    __shared__ alignas(16) uint32_t acc[PERM ? 4 : MAX_BUCKETS];  // this workgroup's ids per bucket, over its tiles
    // A block's run-table columns are staged here, slot s (tile s of the
    // block) at stage[s * STAGE_W + b], and written out as the table's rows,
    // TB contiguous u16 per bucket, when the block ends (up to STAGE_NB
    // buckets; more write the table directly).
    __shared__ alignas(16) uint16_t stage[TB * STAGE_W];
    __shared__ uint32_t lds[4];
    __shared__ uint32_t s_max, s_total;
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
#pragma unroll
            for (uint32_t x = 0; x < 8; ++x) tot->ticket[x] = 0;
        }
    }
    if constexpr (!PERM) {
        for (uint32_t i = t; i < MAX_BUCKETS; i += TS_NT) acc[i] = 0;  // before the barrier ahead of the loop
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
    for (uint32_t i = t; i <= NB; i += TS_NT) cnt[i] = 0;  // the first tile's counts; each tile zeroes the next's
    __syncthreads();
    // The first tile's ids are in before the loop (vmcnt(0)), and every tile
    // ends with the next one's in (below), so the loop's top needs no wait of
    // its own, which would otherwise also wait for the write-out's stores.
    __builtin_amdgcn_s_waitcnt(0x0F70);
    for (uint32_t tile = first; tile < g.n_tiles; tile = next(tile)) {
        // The thread index, opaque to the compiler here, so per-lane addresses
        // are formed inside the loop rather than hoisted out of it and
        // spilled (a spill reload waits for every outstanding load).
        uint32_t t = threadIdx.x;
        asm volatile("" : "+v"(t));
        if (!partial) {
#pragma unroll
            for (uint32_t j = 0; j < TS_PER; ++j) mx = max(mx, v[j]);
        }
        // Ranks within the tile.  A wave whose first and last passes (ids 256
        // apart in a sorted tile) both span several buckets holds random ids:
        // an atomic a lane throughout, with no further test.  Otherwise, when
        // every id of the wave's tile falls in one bucket (clustered ids), a
        // single atomic reserves them all.
        uint32_t rk[TS_PER / 2];  // tile ranks (< 24576) packed two per register
        const uint32_t b00 = __builtin_amdgcn_readfirstlane(bucket(v[0]));
        const uint32_t bl0 = __builtin_amdgcn_readfirstlane(bucket(v[TS_PER - 1]));
        auto one_bucket = [&](uint32_t b) {  // every id of the wave's tile in bucket b
            bool diff = false;
#pragma unroll
            for (uint32_t j = 0; j < TS_PER; ++j) diff |= bucket(v[j]) != b;
            return __ballot(diff) == 0ull;
        };
        if (__ballot(bucket(v[0]) != b00) != 0ull && __ballot(bucket(v[TS_PER - 1]) != bl0) != 0ull) {
#pragma unroll
            for (uint32_t j = 0; j < TS_PER; ++j) {
                const uint32_t r = atomicAdd(&cnt[bucket(v[j])], 1u);
                if (j & 1u)
                    rk[j >> 1] |= r << 16;
                else
                    rk[j >> 1] = r;
            }
        } else if (one_bucket(b00)) {
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
        // Bucket starts: wave w < W scans buckets [1024 w, 1024 w + 1024), 16
        // consecutive ones a lane (four 16-byte LDS reads, one DPP scan), so
        // up to 1024 buckets need no block-wide step.  The pass writes each
        // bucket's start over its count (with PERM the padded start in the
        // high half) and into the tile's slot of the run table (two 16-byte
        // writes when staged); the sentinel bucket NB gets the total, the
        // start of the ids past the universe.  The workgroup's per-bucket
        // totals are taken from the staged starts when a block is written
        // out (unstaged, here).
        {
            const uint32_t W = max(1u, (NB + 1023u) >> 10);  // scanning waves (NB <= 4096)
            const uint32_t wave = t >> 6;
            const uint32_t b0 = 16u * t;  // = 1024 wave + 16 lane
            uint4* c4 = reinterpret_cast<uint4*>(cnt + b0);
            // The counts of the sentinel bucket and past it are left out.  A
            // wave whose buckets are all real (every wave when NB is a multiple
            // of 1024) takes the count as it is: a wave-uniform branch between
            // two copies of each pass, instead of a compare and a select per
            // count on the one wave that the other fifteen wait for.
            const bool whole = __ballot(b0 + 16u > NB) == 0ull;
            auto real = [&](auto masked, uint32_t c, uint32_t b) {
                if constexpr (decltype(masked)::value) return b < NB ? c : 0u;
                else return c;
            };
            auto sum16 = [&](auto masked) {
                uint32_t sum = 0;
#pragma unroll
                for (uint32_t q = 0; q < 4; ++q) {
                    const uint4 c = c4[q];
                    const uint32_t b = b0 + 4u * q;
                    sum += real(masked, c.x, b) + real(masked, c.y, b + 1u) + real(masked, c.z, b + 2u) +
                           real(masked, c.w, b + 3u);
                }
                return sum;
            };
            uint32_t s = 0, incl = 0, seg = 0;
            if (wave < W) {
                if (whole)
                    s = sum16(std::false_type{});
                else
                    s = sum16(std::true_type{});
                incl = wave_incl_scan(s);
                seg = __builtin_amdgcn_readlane(incl, 63);
                if (W > 1u && lane == 63) lds[wave] = seg;
            }
            if (W > 1u) __syncthreads();  // uniform: NB is the workgroup's
            if (wave < W) {
                uint32_t prefix = 0, total_ = seg;
                if (W > 1u) {
                    total_ = 0;
                    for (uint32_t x = 0; x < W; ++x) {
                        const uint32_t y = lds[x];
                        prefix += x < wave ? y : 0u;
                        total_ += y;
                    }
                }
                uint32_t run = prefix + incl - s;
                auto start = [&](uint32_t st, uint32_t b) {
                    return PERM ? st | (((st + 7u * b + 7u) & ~7u) << 16) : st;
                };
                uint32_t st[8];  // the lane's 16 starts as u16 pairs
                auto starts16 = [&](auto masked) {
#pragma unroll
                    for (uint32_t q = 0; q < 4; ++q) {
                        const uint4 c = c4[q];
                        const uint32_t b = b0 + 4u * q;
                        const uint32_t cx = real(masked, c.x, b), cy = real(masked, c.y, b + 1u),
                                       cz = real(masked, c.z, b + 2u), cw = real(masked, c.w, b + 3u);
                        const uint32_t s0 = run, s1 = s0 + cx, s2 = s1 + cy, s3 = s2 + cz;
                        run = s3 + cw;
                        c4[q] = make_uint4(start(s0, b), start(s1, b + 1u), start(s2, b + 2u), start(s3, b + 3u));
                        st[2 * q] = s0 | (s1 << 16);
                        st[2 * q + 1] = s2 | (s3 << 16);
                        if (!staged) {  // straight into the table (entries b <= NB), and the totals
                            uint16_t* rp = tab + (static_cast<uint64_t>(tile / TB) * (NB + 1) + b) * TB + tile % TB;
                            if (b <= NB) rp[0] = static_cast<uint16_t>(s0);
                            if (b + 1u <= NB) rp[TB] = static_cast<uint16_t>(s1);
                            if (b + 2u <= NB) rp[2 * TB] = static_cast<uint16_t>(s2);
                            if (b + 3u <= NB) rp[3 * TB] = static_cast<uint16_t>(s3);
                            if constexpr (!PERM) {
                                uint4* a4 = reinterpret_cast<uint4*>(acc + b);
                                const uint4 a = *a4;
                                *a4 = make_uint4(a.x + cx, a.y + cy, a.z + cz, a.w + cw);
                            }
                        }
                    }
                };
                if (whole)
                    starts16(std::false_type{});
                else
                    starts16(std::true_type{});
                if (staged) {  // W = 1: buckets 16 t .. 16 t + 15 < STAGE_W
                    uint4* sp = reinterpret_cast<uint4*>(stage + (tile % TB) * STAGE_W + b0);
                    sp[0] = make_uint4(st[0], st[1], st[2], st[3]);
                    sp[1] = make_uint4(st[4], st[5], st[6], st[7]);
                }
                // NB a multiple of 1024: the sentinel lies past the last wave's range
                if (wave == W - 1u && lane == 63 && (NB & 1023u) == 0) {
                    cnt[NB] = start(total_, NB);
                    if (staged)
                        stage[(tile % TB) * STAGE_W + NB] = static_cast<uint16_t>(total_);
                    else
                        tab[(static_cast<uint64_t>(tile / TB) * (NB + 1) + NB) * TB + tile % TB] = static_cast<uint16_t>(total_);
                }
                if (t == 0) s_total = total_;
            }
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
            // Nontemporal: read only at the end of the call, in order, and kept
            // out of the Infinity Cache, which then holds the packed tiles.
            if (tile_vec) {  // id j = 4 q + r sits at 4 (t + q TS_NT) + r: one 8-byte store per q
#pragma unroll
                for (uint32_t q = 0; q < TS_PER / 4; ++q)
                    st_stream(reinterpret_cast<uint2*>(pt) + t + q * TS_NT, make_uint2(rk[2 * q], rk[2 * q + 1]));
            } else {  // id j sits at t + j TS_NT
#pragma unroll
                for (uint32_t j = 0; j < TS_PER; ++j)
                    pt[t + j * TS_NT] = static_cast<uint16_t>((rk[j >> 1] >> ((j & 1u) * 16)) & 0xFFFFu);
            }
        }
        __syncthreads();
        const uint32_t total = s_total;  // ids of the real buckets; the sentinel's follow
        for (uint32_t i = t; i <= NB; i += TS_NT) cnt[i] = 0;  // for the next tile's ranks
        if (staged && (tile % TB == TB - 1 || tile + 1 == g.n_tiles)) {
            // The block's rows (TB starts of bucket i, 16 contiguous bytes), and
            // the ids of its tiles in each bucket, start[i + 1] - start[i],
            // added to the workgroup's totals (slots past the block's last
            // tile hold nothing of it).
            uint4* trow = reinterpret_cast<uint4*>(tab + static_cast<uint64_t>(tile / TB) * (NB + 1) * TB);
            const uint32_t used = tile % TB + 1u;
            for (uint32_t i = t; i <= NB; i += TS_NT) {
                uint32_t r[TB];
#pragma unroll
                for (uint32_t sl = 0; sl < TB; ++sl) r[sl] = stage[sl * STAGE_W + i];
                trow[i] = make_uint4(r[0] | (r[1] << 16), r[2] | (r[3] << 16), r[4] | (r[5] << 16), r[6] | (r[7] << 16));
                if constexpr (!PERM) {
                    if (i < NB) {
                        uint32_t n = 0;
#pragma unroll
                        for (uint32_t sl = 0; sl < TB; ++sl)
                            n += sl < used ? static_cast<uint32_t>(stage[sl * STAGE_W + i + 1u]) - r[sl] : 0u;
                        acc[i] += n;
                    }
                }
            }
        }
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
        __syncthreads();  // also: the counts are zeroed for the next tile's ranks
#pragma unroll
        for (uint32_t k = 0; k < GPT; ++k)
#pragma unroll
            for (uint32_t q = 0; q < 5u; ++q) buf[5u * (t + k * TS_NT) + q] = pw[k][q];
        __syncthreads();
        uint4* dst = reinterpret_cast<uint4*>(part + static_cast<uint64_t>(tile) * TILE_WORDS);
        const uint32_t n4 = (FIELD_BITS * total + 127u) >> 7;
        // Ordinary stores, so the packed tiles are kept in the Infinity Cache
        // for the kernel that reads them next; the ids come in through
        // nontemporal loads, which do not displace them.  The next tile's
        // scatter overwrites buf only after two more barriers.  Every lane
        // makes the same number of stores (one past the last vector stores
        // that vector again, the same bytes; a tile without real ids writes
        // its slot's first vector, which no run covers): the memory counter
        // counts stores with loads, in order, so with a fixed count the next
        // tile waits for its ids alone and leaves these stores in flight.
        constexpr uint32_t WO = (TILE_WORDS / 4 + TS_NT - 1) / TS_NT;  // 16-byte vectors a lane
        const uint32_t last = max(n4, 1u) - 1u;
        uint4 wv[WO];
#pragma unroll
        for (uint32_t k = 0; k < WO; ++k) wv[k] = reinterpret_cast<const uint4*>(buf)[min(t + k * TS_NT, last)];
#pragma unroll
        for (uint32_t k = 0; k < WO; ++k) dst[min(t + k * TS_NT, last)] = wv[k];
        // vmcnt(WO): the next tile's ids, loaded before these WO stores, are in.
        static_assert(WO == 4, "the wait below counts WO stores");
        __builtin_amdgcn_s_waitcnt(0x0F74);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = max(mx, static_cast<uint32_t>(__shfl_xor(mx, o, 64)));
    if (lane == 0) atomicMax(&s_max, mx);
    __syncthreads();
    if (t == 0) gmax[blockIdx.x] = s_max;  // per-workgroup partials: nothing here needs zeroed memory
    if (!PERM && wg_count != nullptr)
        for (uint32_t i = t; i < NB; i += TS_NT) wg_count[static_cast<uint64_t>(blockIdx.x) * NB + i] = acc[i];
}

constexpr int BUILD_NT = 1024;
constexpr uint32_t BUILD_WAVES = BUILD_NT / 64;

// Workgroups go round-robin over the 8 XCDs; XCD x takes the contiguous
// bucket range [x * per, (x + 1) * per), in order, so almost every pair of
// neighbouring buckets -- whose runs share the cache line at their boundary in
// every tile -- runs on one XCD, close in time, and that line comes from its L2.
__host__ __device__ inline uint32_t build_per_xcd(uint32_t nb) { return (nb + 7) / 8; }
inline uint32_t build_grid(uint32_t nb) { return 8 * build_per_xcd(nb); }
// The persistent build: up to one workgroup per CU, none without a bucket.
inline uint32_t build_grid_persistent(uint32_t nb, uint32_t cus)
{
    return 8 * std::min(build_per_xcd(nb), std::max(1u, cus / 8));
}

// Calls on_group(tile, p, n, f) for every group of 8 consecutive fields of
// bucket b's run in every tile: the run holds sorted positions [S, E) of the
// tile, a group the fields p .. p + 7 with p = S + 8 j, of which the first
// n = min(8, E - p) are the run's (the rest are whatever follows in the tile's
// stream, possibly past what the tile sort wrote: any 20-bit value); f[k] is
// field k's 20 bits, unmasked above them.  n = 0 marks an empty slot of a
// round, whose fields are any of the tile's: on_group must then leave no trace.  prologue() runs first, in every
// thread, once the first run bounds are requested: the caller's LDS set-up,
// published by a workgroup barrier before the first on_group.  Every thread of
// the BUILD_NT-thread workgroup calls it (wave = t >> 6, lane = its lane).
// A group's reads are the 6 words from its first word on: `part` needs 8
// words of slack past the last tile.
//
// Wave w owns tile blocks w, w + 16, ...; a step covers 2 x 64 / TB of them,
// two tiles per lane, whose run bounds are loaded a step ahead.  The step's
// groups are numbered across the wave (an exclusive scan of the lanes' group
// counts); each lane writes a 4-byte descriptor of each of its groups into the
// wave's LDS list `desc` (DESC_CAP entries: longer steps go in chunks), and the
// lanes then take the groups in rounds of 64, lane l the l-th of each round, so
// neighbouring lanes read neighbouring words of one run (their loads share
// cache lines); eight rounds are loaded before any is handed on.  A descriptor
// is the owner lane (6 bits), which of its two tiles (1), the group's first
// sorted position p (15: p < TILE), n - 1 (3) and the first field's bit in its
// word, 20 p mod 32 (5: the same for every group of a run, 8 fields being 5
// words).  A run of more than GROUP_LONG groups (sorted or clustered ids: a
// bucket's fields in a few tiles, all in one wave's blocks) is queued in LDS
// and its groups dealt to all sixteen waves after the walk; one that finds the
// queue full is dealt with its wave's other runs.  `queue` is the workgroup's
// LDS queue.
constexpr uint32_t GROUP_LONG = 64;
constexpr uint32_t GROUP_QCAP = 1024;  // 8 KiB of LDS beside the callers' 128 KiB image
constexpr uint32_t DESC_CAP = 256;     // descriptors per wave: 16 KiB for sixteen waves
constexpr uint32_t DESC_EMPTY = 1u << 31;  // a round's slot past the step's last group (n = 0)
constexpr uint32_t DESC_ROUNDS = DESC_CAP / 64;  // rounds of 64 groups the list holds
constexpr uint32_t WALK_ROUNDS = 2 * DESC_ROUNDS;   // groups a lane has in flight
static_assert(TILE <= 32768, "descriptor positions are 15 bits");

// LDS queue of long runs, declared by walk_groups' caller: one per
// workgroup, whatever the number of walk_groups instances it inlines.
struct GroupQueue {
    uint2 ent[GROUP_QCAP];  // {tile, S | E << 16}
    uint32_t n;
};

struct FieldGroup {
    uint32_t x[6];  // words w0 .. w0 + 5
    uint32_t o;     // the first field's bit within word w0
};

// Two words at any 4-byte boundary: the hardware takes a multi-dword global
// load at dword alignment, so a group is read from its own first word.
typedef uint32_t u32x2_dw __attribute__((ext_vector_type(2), aligned(4)));

// The words of the group whose first field sits at sorted position p of
// `tile`: three 8-byte loads from w0, the word holding the first field.
struct GroupWords {
    u32x2_dw p[3];
    uint32_t o;
};

// The word of `part` holding the first field of the group at sorted position p
// of `tile`: tile * TILE_WORDS + 20 p / 32, below 2^32 since the callers take
// at most 0xFFFFFFFF / TILE_WORDS tiles (24-bit multiplies: full rate).
__device__ __forceinline__ uint32_t group_word(uint32_t tile, uint32_t p)
{
    return __umul24(tile, TILE_WORDS) + (__umul24(FIELD_BITS, p) >> 5);
}

__device__ __forceinline__ void group_issue(const uint32_t* __restrict__ part, uint32_t tile, uint32_t p,
                                            GroupWords& q)
{
    q.o = __umul24(FIELD_BITS, p) & 31u;
    const u32x2_dw* src = reinterpret_cast<const u32x2_dw*>(part + group_word(tile, p));
#pragma unroll
    for (int i = 0; i < 3; ++i) q.p[i] = src[i];
}

__device__ __forceinline__ void group_words(const GroupWords& w, FieldGroup& q)
{
    q.x[0] = w.p[0].x, q.x[1] = w.p[0].y, q.x[2] = w.p[1].x;
    q.x[3] = w.p[1].y, q.x[4] = w.p[2].x, q.x[5] = w.p[2].y;
    q.o = w.o;
}

__device__ __forceinline__ void group_fields(const FieldGroup& q, uint32_t (&f)[8])
{
    static_assert(FIELD_BITS == 20, "8 fields = 5 words");
    const uint32_t d0 = __builtin_amdgcn_alignbit(q.x[1], q.x[0], q.o);
    const uint32_t d1 = __builtin_amdgcn_alignbit(q.x[2], q.x[1], q.o);
    const uint32_t d2 = __builtin_amdgcn_alignbit(q.x[3], q.x[2], q.o);
    const uint32_t d3 = __builtin_amdgcn_alignbit(q.x[4], q.x[3], q.o);
    const uint32_t d4 = __builtin_amdgcn_alignbit(q.x[5], q.x[4], q.o);
    f[0] = d0;
    f[1] = __builtin_amdgcn_alignbit(d1, d0, 20);
    f[2] = d1 >> 8;
    f[3] = __builtin_amdgcn_alignbit(d2, d1, 28);
    f[4] = __builtin_amdgcn_alignbit(d3, d2, 16);
    f[5] = d3 >> 4;
    f[6] = __builtin_amdgcn_alignbit(d4, d3, 24);
    f[7] = d4 >> 12;
}

// WHOLE_TAIL (an on_group for which a field seen twice is the same as once,
// such as setting its bit): a run of at least 8 fields ends in a whole group,
// fields E - 8 .. E - 1, which repeats some of the group before it, so only
// runs shorter than 8 fields hand on_group a partial group.
template <bool WHOLE_TAIL, class Prologue, class OnGroup>
__device__ __forceinline__ void walk_groups(const uint32_t* __restrict__ part, const uint16_t* __restrict__ tab,
                                            const IdsGeom& g, uint32_t b, uint32_t wave, uint32_t lane,
                                            GroupQueue& queue, uint32_t* desc, Prologue prologue, OnGroup on_group)
{
    uint2* q_ent = queue.ent;
    uint32_t& q_n = queue.n;
    auto handle = [&](uint32_t tile, uint32_t p, uint32_t n, const GroupWords& w) {
        FieldGroup q;
        group_words(w, q);
        uint32_t f[8];
        group_fields(q, f);
        on_group(tile, p, n, f);
    };
    constexpr uint32_t BPS = 64u / TB;
    const uint32_t n_blk = (g.n_tiles + TB - 1) / TB;
    const uint32_t per_wave = n_blk > wave ? (n_blk - wave + BUILD_WAVES - 1) / BUILD_WAVES : 0u;
    auto tile_of = [&](uint32_t st, uint32_t l) { return (wave + BUILD_WAVES * (st * BPS + l / TB)) * TB + l % TB; };
    // tile_of(2 st + a, l) for a descriptor's owner lane l (bits 0-5) and tile a
    // (bit 6): with TB = BPS = 8, (2 st + a) BPS + l / TB = 16 st + bits 3-6.
    static_assert(TB == 8 && BPS == 8, "desc_tile's bit fields");
    auto desc_tile = [&](uint32_t st, uint32_t d) {
        return wave * TB + BUILD_WAVES * TB * (16u * st + ((d >> 3) & 15u)) + (d & 7u);
    };
    auto tab_load = [&](uint32_t st, uint32_t& r0, uint32_t& r1) {
        r0 = r1 = 0;
        const uint32_t jb = st * BPS + lane / TB;
        if (jb < per_wave && tile_of(st, lane) < g.n_tiles) {
            const uint16_t* tc =
                tab + (static_cast<uint64_t>(wave + BUILD_WAVES * jb) * (g.NB + 1) + b) * TB + lane % TB;
            r0 = tc[0];
            r1 = tc[TB];
        }
    };
    uint32_t* wdesc = desc + wave * DESC_CAP;
    uint32_t a0, a1, b0, b1;
    tab_load(0, a0, a1);
    tab_load(1, b0, b1);
    // The caller's set-up of its LDS (the first run bounds are in flight
    // meanwhile); the barrier publishes it.
    prologue();
    if (threadIdx.x == 0) q_n = 0;
    __syncthreads();
    for (uint32_t st = 0; 2u * st * BPS < per_wave; ++st) {
        const uint32_t Sa = a0, Ea = a1, Sb = b0, Eb = b1;
        tab_load(2u * st + 2u, a0, a1);
        tab_load(2u * st + 3u, b0, b1);
        uint32_t Ga = (Ea - Sa + 7u) / 8u, Gb = (Eb - Sb + 7u) / 8u;  // E >= S
        if (Ga > GROUP_LONG) {
            const uint32_t slot = atomicAdd(&q_n, 1u);
            if (slot < GROUP_QCAP) q_ent[slot] = make_uint2(tile_of(2u * st, lane), Sa | (Ea << 16)), Ga = 0;
        }
        if (Gb > GROUP_LONG) {
            const uint32_t slot = atomicAdd(&q_n, 1u);
            if (slot < GROUP_QCAP) q_ent[slot] = make_uint2(tile_of(2u * st + 1u, lane), Sb | (Eb << 16)), Gb = 0;
        }
        const uint32_t G = Ga + Gb;
        uint32_t P = wave_incl_scan(G);  // then exclusive: the lane's first group
        const uint32_t T = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(P), 63));
        P -= G;
        // Writes the descriptors of a run's groups that fall in the list's
        // window [w0, w0 + DESC_CAP): group j (numbered `first` + j) of a run
        // at [S, E) starts at p = S + 8 j, so a whole group's descriptor is
        // the first one's plus 1024 j; the last group's n, and with
        // WHOLE_TAIL its p and bit, are written over it afterwards (the same
        // lane's LDS writes land in order).
        auto put_run = [&](uint32_t w0, uint32_t first, uint32_t Gr, uint32_t S, uint32_t E, uint32_t which) {
            if (Gr == 0u) return;
            const uint32_t d0 = lane | which | (S << 7) | (7u << 22) | ((__umul24(FIELD_BITS, S) & 31u) << 25);
            const uint32_t hi = min(first + Gr, w0 + DESC_CAP);
            for (uint32_t u = max(first, w0); u < hi; ++u) wdesc[u - w0] = d0 + ((u - first) << 10);
            const uint32_t ul = first + Gr - 1u;
            if (ul - w0 < DESC_CAP) {
                uint32_t p = S + 8u * (Gr - 1u), n = E - p;  // 1 .. 8
                // the whole tail's bit: 20 (E - 8) mod 32 = 20 E mod 32
                if (WHOLE_TAIL && n < 8u && E - S >= 8u) p = E - 8u, n = 8u;
                wdesc[ul - w0] = lane | which | (p << 7) | ((n - 1u) << 22) | ((__umul24(FIELD_BITS, p) & 31u) << 25);
            }
        };
        // Batches of WALK_ROUNDS rounds (64 groups a round): the descriptor
        // list holds DESC_ROUNDS rounds, so it is filled and read into
        // registers WALK_ROUNDS / DESC_ROUNDS times per batch before any load.
        for (uint32_t c0 = 0; c0 < T; c0 += 64u * WALK_ROUNDS) {
            uint32_t dd[WALK_ROUNDS];
#pragma unroll
            for (uint32_t h = 0; h < WALK_ROUNDS / DESC_ROUNDS; ++h) {
                const uint32_t w0 = c0 + h * DESC_CAP;  // wave-uniform
                if (w0 < T) {
                    // This lane's groups numbered [w0, w0 + DESC_CAP): their descriptors.
                    put_run(w0, P, Ga, Sa, Ea, 0u);
                    put_run(w0, P + Ga, Gb, Sb, Eb, 64u);
                    wave_lds_fence();
#pragma unroll
                    for (uint32_t k = 0; k < DESC_ROUNDS; ++k) {
                        const uint32_t u = w0 + 64u * k + lane;
                        // an empty slot repeats the step's last group, marked empty
                        dd[h * DESC_ROUNDS + k] = wdesc[min(u, T - 1u) - w0] | (u < T ? 0u : DESC_EMPTY);
                    }
                    wave_lds_fence();  // the reads are done before the list is written again
                } else {
#pragma unroll
                    for (uint32_t k = 0; k < DESC_ROUNDS; ++k) dd[h * DESC_ROUNDS + k] = dd[h * DESC_ROUNDS - 1u] | DESC_EMPTY;
                }
            }
            // All the batch's addresses, then all its loads, then the groups:
            // no branch between, so the loads are in flight together.
            const u32x2_dw* src[WALK_ROUNDS];
#pragma unroll
            for (uint32_t k = 0; k < WALK_ROUNDS; ++k)
                src[k] = reinterpret_cast<const u32x2_dw*>(part + group_word(desc_tile(st, dd[k]), (dd[k] >> 7) & 0x7FFFu));
            GroupWords w[WALK_ROUNDS];
#pragma unroll
            for (uint32_t k = 0; k < WALK_ROUNDS; ++k)
#pragma unroll
                for (int i = 0; i < 3; ++i) w[k].p[i] = src[k][i];
#pragma unroll
            for (uint32_t k = 0; k < WALK_ROUNDS; ++k) {
                const uint32_t p = (dd[k] >> 7) & 0x7FFFu;
                w[k].o = (dd[k] >> 25) & 31u;
                const uint32_t tile = desc_tile(st, dd[k]);
                handle(tile, p, (dd[k] & DESC_EMPTY) ? 0u : ((dd[k] >> 22) & 7u) + 1u, w[k]);
            }
        }
    }
    // The queued runs: their groups in chunks of 64 (one a lane), the chunks of
    // all runs dealt to the waves in turn.
    __syncthreads();
    const uint32_t nq = min(q_n, GROUP_QCAP);
    uint32_t off = 0;
    for (uint32_t i = 0; i < nq; ++i) {
        const uint2 ent = q_ent[i];
        const uint32_t S = ent.y & 0xFFFFu, E = ent.y >> 16;
        const uint32_t G = (E - S + 7u) / 8u;
        const uint32_t nch = (G + 63u) / 64u;
        for (uint32_t c = (wave + BUILD_WAVES - off % BUILD_WAVES) % BUILD_WAVES; c < nch; c += BUILD_WAVES) {
            const uint32_t j = 64u * c + lane;
            if (j < G) {
                uint32_t p = S + 8u * j, n = min(E - p, 8u);
                if (WHOLE_TAIL && n < 8u && E - S >= 8u) p = E - 8u, n = 8u;
                GroupWords w;
                group_issue(part, ent.x, p, w);
                handle(ent.x, p, n, w);
            }
        }
        off += nch;
    }
}

}  // namespace crimpl

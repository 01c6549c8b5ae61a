// Batched point queries over the header-only device API.
//
// The reference's benches wrap view.contains() / warp_contains() in one-query-
// per-thread kernels (bench/bench_point_query.cu:123-144).  Here each lane
// keeps QPT independent queries in flight so the dependent key_index -> word
// loads of different queries overlap (random queries are latency-bound gathers
// from the 256 MB Infinity Cache / HBM).  Modes 0 and 1 on an all-bitmap view
// take the view's two-load fast path written without branches; on other
// layouts mode 0 calls GpuRoaringView::contains and mode 1 runs a lockstep
// search of each lane's queries; modes 2 and 3, on every layout, call
// GpuRoaringView::contains and wavefront_contains unchanged.
#include <algorithm>
#include <cstring>

#include "cu_roaring/device/roaring_view.hpp"
#include "cu_roaring/device/roaring_wavefront_query.hpp"
#include "internal.hpp"
#include "tiles.hpp"

namespace crimpl {

using cu_roaring::GpuRoaringView;

constexpr int Q_NT = 256;
constexpr int QPT = 8;

// The id stream and the answers use nontemporal loads and stores, so they do
// not evict the containers (reused by every query) from the caches.
// WAVE: when every lane of the wave queries the same key, the key_index entry
// is read once with a wave-uniform (scalar) load -- wavefront_contains'
// amortisation -- while the QPT queries of a lane stay independent.
template <bool WAVE>
__global__ __launch_bounds__(Q_NT) void contains_allbitmap(GpuRoaringView v, const uint32_t* __restrict__ ids,
                                                           uint64_t n, uint32_t* __restrict__ out)
{
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * Q_NT * QPT;
    const uint32_t neg = v.negated ? 1u : 0u;
    for (uint64_t blk = static_cast<uint64_t>(blockIdx.x) * Q_NT * QPT; blk < n; blk += stride) {
        uint32_t id[QPT], idx[QPT];
#pragma unroll
        for (int q = 0; q < QPT; ++q) {
            const uint64_t i = blk + static_cast<uint64_t>(q) * Q_NT + threadIdx.x;
            id[q] = i < n ? __builtin_nontemporal_load(ids + i) : 0u;
        }
#pragma unroll
        for (int q = 0; q < QPT; ++q) {
            const uint32_t key = id[q] >> 16;
            if (WAVE) {
                const uint32_t k0 = __builtin_amdgcn_readfirstlane(key);
                if (__ballot(key != k0) == 0ull) {  // wave-uniform key
                    const uint32_t x = v.key_index[min(k0, v.max_key)];
                    idx[q] = k0 > v.max_key ? 0xFFFFu : x;
                    continue;
                }
            }
            const uint32_t k = min(key, v.max_key);
            const uint32_t x = v.key_index[k];
            idx[q] = key > v.max_key ? 0xFFFFu : x;
        }
#pragma unroll
        for (int q = 0; q < QPT; ++q) {
            const uint64_t i = blk + static_cast<uint64_t>(q) * Q_NT + threadIdx.x;
            uint32_t r = neg;
            if (idx[q] != 0xFFFFu) {
                const uint32_t low = id[q] & 0xFFFFu;
                const uint64_t w = v.bitmap_data[(idx[q] << 10) + (low >> 6)];
                r = (static_cast<uint32_t>(w >> (low & 63u)) & 1u) ^ neg;
            }
            if (i < n) __builtin_nontemporal_store(r, out + i);
        }
    }
}

// Mode 1 on a view that is not all-bitmap, for wave-coherent (clustered)
// batches: each lane answers QI queries by contains()'s rules (key lookup
// through key_index or a search of keys, then one bitset word, or a search of
// an array's values or a run container's starts), with the QI lookups advanced
// in lockstep -- every step issues QI independent loads, so a lane's dependent
// chains overlap instead of running one query after another, and a wave whose
// q-th queries share one key reads its key_index entry with one wave-uniform
// load (wavefront_contains' saving).  Searches are lower bounds over sorted u16
// sequences (element i at base + step * i): an array's first value >= low, a
// run container's first start > low (the run before it holds low iff low <=
// start + length), the keys' first key >= key.
// Measured at 2^30 on 16384 array containers: clustered queries 198 Gq/s
// (0.1%) and 161 (1%) against 102 and 77 for wavefront_contains one query at a
// time; on uniform queries, which are bound by the L2's request rate rather
// than by latency, lockstep searching loses (7.6 against 11.8 Gq/s at 1%), so
// mode 0 keeps the header function there.  QI = 4 measured above 2, 8 and 16.
constexpr int QI = 4;

__global__ __launch_bounds__(Q_NT) void contains_interleaved(GpuRoaringView v, const uint32_t* __restrict__ ids,
                                                             uint64_t n, uint32_t* __restrict__ out)
{
    using cu_roaring::ContainerTypeD;
    constexpr int QPT = QI;
    constexpr bool WAVE = true;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * Q_NT * QPT;
    const uint32_t neg = v.negated ? 1u : 0u;
    // Lockstep lower bounds: lo[q] ends at the first index whose element is >= tgt[q].
    auto lower_bounds = [](const uint16_t* const (&base)[QPT], const uint32_t (&step)[QPT], uint32_t (&len)[QPT],
                           const uint32_t (&tgt)[QPT], uint32_t (&lo)[QPT]) {
        for (;;) {
            bool any = false;
#pragma unroll
            for (int q = 0; q < QPT; ++q) any |= len[q] > 0u;
            if (!any) break;
            uint32_t x[QPT];
#pragma unroll
            for (int q = 0; q < QPT; ++q) x[q] = len[q] > 0u ? base[q][step[q] * (lo[q] + (len[q] >> 1))] : 0u;
#pragma unroll
            for (int q = 0; q < QPT; ++q) {
                const uint32_t half = len[q] >> 1;
                if (len[q] > 0u && x[q] < tgt[q]) {
                    lo[q] += half + 1u;
                    len[q] -= half + 1u;
                } else {
                    len[q] = half;
                }
            }
        }
    };
    for (uint64_t blk = static_cast<uint64_t>(blockIdx.x) * Q_NT * QPT; blk < n; blk += stride) {
        uint32_t id[QPT], idx[QPT];  // idx: container index, 0xFFFFFFFF = absent
#pragma unroll
        for (int q = 0; q < QPT; ++q) {
            const uint64_t i = blk + static_cast<uint64_t>(q) * Q_NT + threadIdx.x;
            id[q] = i < n ? __builtin_nontemporal_load(ids + i) : 0u;
        }
        if (v.key_index) {
#pragma unroll
            for (int q = 0; q < QPT; ++q) {
                const uint32_t key = id[q] >> 16;
                const uint32_t k0 = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(key));
                uint32_t x;
                if (WAVE && __ballot(key != k0) == 0ull)
                    x = v.key_index[min(k0, v.max_key)];
                else
                    x = v.key_index[min(key, v.max_key)];
                idx[q] = (key > v.max_key || x == 0xFFFFu) ? 0xFFFFFFFFu : x;
            }
        } else {
            const uint16_t* base[QPT];
            uint32_t step[QPT], len[QPT], tgt[QPT], lo[QPT];
#pragma unroll
            for (int q = 0; q < QPT; ++q) {
                base[q] = v.keys, step[q] = 1u, len[q] = v.n_containers, tgt[q] = id[q] >> 16, lo[q] = 0u;
            }
            lower_bounds(base, step, len, tgt, lo);
#pragma unroll
            for (int q = 0; q < QPT; ++q)
                idx[q] = (lo[q] < v.n_containers && v.keys[lo[q]] == tgt[q]) ? lo[q] : 0xFFFFFFFFu;
        }
        uint32_t type[QPT], card[QPT], off[QPT];
#pragma unroll
        for (int q = 0; q < QPT; ++q) {
            const bool hit = idx[q] != 0xFFFFFFFFu;
            type[q] = hit ? static_cast<uint32_t>(v.types[idx[q]]) : 0xFFu;
            off[q] = hit ? v.offsets[idx[q]] : 0u;
            card[q] = hit ? v.cardinalities[idx[q]] : 0u;
        }
        const uint16_t* base[QPT];
        uint32_t step[QPT], len[QPT], tgt[QPT], lo[QPT], r[QPT];
#pragma unroll
        for (int q = 0; q < QPT; ++q) {
            const uint32_t low = id[q] & 0xFFFFu;
            const bool arr = type[q] == static_cast<uint32_t>(ContainerTypeD::ARRAY);
            const bool run = type[q] == static_cast<uint32_t>(ContainerTypeD::RUN);
            base[q] = arr ? v.array_data + (off[q] >> 1) : v.run_data + (off[q] >> 1);
            step[q] = run ? 2u : 1u;
            len[q] = (arr || run) ? card[q] : 0u;
            tgt[q] = run ? low + 1u : low;
            lo[q] = 0u;
            r[q] = 0u;
            if (type[q] == static_cast<uint32_t>(ContainerTypeD::BITMAP)) {
                const uint64_t w = v.bitmap_data[(off[q] >> 3) + (low >> 6)];
                r[q] = static_cast<uint32_t>(w >> (low & 63u)) & 1u;
            }
        }
        lower_bounds(base, step, len, tgt, lo);
#pragma unroll
        for (int q = 0; q < QPT; ++q) {
            const uint32_t low = id[q] & 0xFFFFu;
            if (type[q] == static_cast<uint32_t>(ContainerTypeD::ARRAY)) {
                r[q] = lo[q] < card[q] && base[q][lo[q]] == low;
            } else if (type[q] == static_cast<uint32_t>(ContainerTypeD::RUN) && lo[q] > 0u) {
                const uint16_t* rr = base[q] + 2u * (lo[q] - 1u);
                r[q] = low <= static_cast<uint32_t>(rr[0]) + rr[1];
            }
            const uint64_t i = blk + static_cast<uint64_t>(q) * Q_NT + threadIdx.x;
            if (i < n) __builtin_nontemporal_store(r[q] ^ neg, out + i);
        }
    }
}

template <int MODE>
__global__ __launch_bounds__(Q_NT) void contains_general(GpuRoaringView v, const uint32_t* __restrict__ ids,
                                                         uint64_t n, uint32_t* __restrict__ out)
{
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * Q_NT * QPT;
    for (uint64_t blk = static_cast<uint64_t>(blockIdx.x) * Q_NT * QPT; blk < n; blk += stride) {
#pragma unroll
        for (int q = 0; q < QPT; ++q) {
            const uint64_t i = blk + static_cast<uint64_t>(q) * Q_NT + threadIdx.x;
            if (i < n) {
                const uint32_t id = __builtin_nontemporal_load(ids + i);
                const bool r = MODE == CR_QUERY_WAVEFRONT ? cu_roaring::wavefront_contains(v, id) : v.contains(id);
                __builtin_nontemporal_store(r ? 1u : 0u, out + i);
            }
        }
    }
}

// ---- partitioned point queries (CR_QUERY_PARTITIONED) ----------------------------
// Uniform random queries over a large bitmap are bound by the memory system's
// random-request rate: every query is one dependent read of a cache line (100M
// queries = 100M fabric read requests).  Partitioned, the same answers cost a
// few streaming bytes per query and one read of each container:
//   ids_tile_sort<true>  tile-sort the query ids by 16-key bucket (the
//                        upload's tile sort), recording each query's padded
//                        sorted position within its tile (perm, u16);
//   qp_answer            one workgroup per bucket loads the bucket's 16
//                        containers into LDS as bitmaps and answers every query
//                        of the bucket from LDS: a bit at its padded sorted
//                        position, eight answers to a byte;
//   qp_unpermute         one workgroup per tile stages the tile's answer bits
//                        in LDS and writes out[i] = answer[perm[i]] in input
//                        order.
// A query whose key lies past the bitmap's last bucket (sorted into the tile
// sort's sentinel run) answers `negated`, as contains() does for key > max_key.

// Answer-bit layout of a tile (see qp_answer): bucket b's run starting at
// sorted position S is answered from bit qp_pstart(S, b); a tile's bits take
// qp_abytes(NB) bytes (16-byte multiple), at most QA_MAX_ABYTES.
__host__ __device__ inline uint32_t qp_pstart(uint32_t s, uint32_t b) { return (s + 7u * b + 7u) & ~7u; }
__host__ __device__ inline uint32_t qp_abytes(uint32_t nb)
{
    return ((TILE + 7u * nb + 7u + 7u) / 8u + 15u) & ~15u;  // the sentinel run ends below TILE + 7 NB + 7
}
constexpr uint32_t QA_MAX_ABYTES = ((TILE + 7u * MAX_BUCKETS + 14u) / 8u + 15u) & ~15u;

// One wave fills `w` (2048 words) with key's container as a bitmap -- zeros
// when the key is absent -- found by contains()'s own lookup rules.
__device__ void qp_load_container(const GpuRoaringView& v, uint32_t key, uint32_t* w, uint32_t lane)
{
    int idx = -1;
    if (v.all_bitmap) {
        if (key <= v.max_key) {
            const uint32_t x = v.key_index[key];
            idx = x == 0xFFFFu ? -1 : static_cast<int>(x);
        }
    } else {
        idx = v.lookup_key(key);
    }
    uint4* w4 = reinterpret_cast<uint4*>(w);
    uint32_t type = CR_BITMAP, off = 0, card = 0;
    if (idx >= 0 && !v.all_bitmap) {
        type = static_cast<uint32_t>(v.types[idx]);
        off = v.offsets[idx];
        card = v.cardinalities[idx];
    }
    if (idx >= 0 && type == CR_BITMAP) {
        const uint64_t* src = v.all_bitmap ? v.bitmap_data + (static_cast<uint64_t>(idx) << 10) : v.bitmap_data + (off >> 3);
        if ((reinterpret_cast<uintptr_t>(src) & 15u) == 0) {
            uint4 x[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) x[j] = ld_stream(reinterpret_cast<const uint4*>(src) + lane + 64 * j);
#pragma unroll
            for (int j = 0; j < 8; ++j) w4[lane + 64 * j] = x[j];
        } else {
            const uint32_t* s32 = reinterpret_cast<const uint32_t*>(src);
            for (uint32_t i = lane; i < 2048u; i += 64) w[i] = s32[i];
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) w4[lane + 64 * j] = make_uint4(0, 0, 0, 0);
    if (idx < 0) return;
    if (type == CR_ARRAY) {  // the wave's LDS operations retire in order: the zeros land first
        const uint16_t* arr = v.array_data + (off >> 1);
        for (uint32_t i0 = lane; i0 < card; i0 += 8u * 64u) {  // eight values a lane in flight
            uint32_t x[8];
#pragma unroll
            for (uint32_t k = 0; k < 8u; ++k) x[k] = i0 + 64u * k < card ? static_cast<uint32_t>(arr[i0 + 64u * k]) : ~0u;
#pragma unroll
            for (uint32_t k = 0; k < 8u; ++k)
                if (x[k] != ~0u) atomicOr(&w[x[k] >> 5], 1u << (x[k] & 31u));
        }
    } else if (type == CR_RUN) {
        // Lane l owns words [32 l, 32 l + 32) (bits [1024 l, 1024 l + 1024)):
        // a binary search finds the first run ending at or after them, then the
        // sorted runs that overlap them set their bits.  Ends are clamped to
        // 0xFFFF, as contains() accepts any low <= 0xFFFF past a run's start.
        const uint16_t* runs = v.run_data + (off >> 1);
        const uint32_t lo = 1024u * lane, hi = lo + 1023u;
        int a = 0, z = static_cast<int>(card);  // first run with start + len >= lo
        while (a < z) {
            const int mid = (a + z) >> 1;
            if (static_cast<uint32_t>(runs[2 * mid]) + runs[2 * mid + 1] < lo)
                a = mid + 1;
            else
                z = mid;
        }
        for (uint32_t r = static_cast<uint32_t>(a); r < card; ++r) {
            const uint32_t s = runs[2 * r];
            if (s > hi) break;
            const uint32_t e = min(min(0xFFFFu, s + runs[2 * r + 1]), hi);
            const uint32_t b0 = max(s, lo);
            for (uint32_t x = b0; x <= e;) {  // word by word within the lane's range
                const uint32_t wi = x >> 5, sb = x & 31u;
                const uint32_t eb = min(31u, e - (x & ~31u));
                w[wi] |= (eb - sb == 31u ? ~0u : ((1u << (eb - sb + 1u)) - 1u)) << sb;
                x = (wi + 1u) << 5;
            }
        }
    }
}

// The answers of a tile are bits at *padded* positions: bucket b's run of the
// tile, sorted positions [S, S + C), is answered at [P, P + C) with
// P = qp_pstart(S, b), a multiple of 8, and the bits up to the next bucket's
// start belong to b as well.  So a lane that answers 8 consecutive fields of
// one run writes one whole byte that no other lane writes (no partial stores,
// one store per 8 queries).  ids_tile_sort<true> records each query's padded
// position in perm.
__global__ __launch_bounds__(BUILD_NT) void qp_answer(const uint32_t* __restrict__ part,
                                                      const uint16_t* __restrict__ tab, IdsGeom g, GpuRoaringView v,
                                                      uint8_t* __restrict__ ans)
{
    __shared__ alignas(16) uint32_t bits[BK_KEYS * 2048u];  // the bucket's 16 containers, 128 KiB
    __shared__ GroupQueue queue;
    __shared__ uint32_t desc[BUILD_WAVES * DESC_CAP];
    const uint32_t t = threadIdx.x;
    const uint32_t b = (blockIdx.x % 8) * build_per_xcd(g.NB) + blockIdx.x / 8;
    if (b >= g.NB) return;
    const uint32_t wave = t >> 6, lane = __lane_id();
    const uint32_t key = b * BK_KEYS + wave;
    const uint32_t flip = v.negated ? 0xFFu : 0u;
    const uint32_t abytes = qp_abytes(g.NB);
    // All 8 answers of a group go into one byte that only this lane writes:
    // fields past the run answer into b's padding, and any 20-bit value
    // indexes the LDS image.
    walk_groups<false>(part, tab, g, b, wave, lane, queue, desc,
                [&] {  // wave w loads container w of the bucket (zeros past the last key)
                    if (key < g.K) {
                        qp_load_container(v, key, bits + wave * 2048u, lane);
                    } else {
                        uint4* w4 = reinterpret_cast<uint4*>(bits + wave * 2048u);
#pragma unroll
                        for (int j = 0; j < 8; ++j) w4[lane + 64 * j] = make_uint4(0, 0, 0, 0);
                    }
                },
                [&](uint32_t tile, uint32_t p, uint32_t n, const uint32_t (&f)[8]) {
                    uint32_t a = 0;
#pragma unroll
                    for (uint32_t k = 0; k < 8u; ++k) {
                        const uint32_t F = f[k] & FIELD_MASK;
                        a |= ((bits[F >> 5] >> (F & 31u)) & 1u) << k;
                    }
                    // p = S + 8 j for the run's start S: qp_pstart(p, b) = qp_pstart(S, b) + 8 j
                    if (n != 0u)
                        ans[static_cast<uint64_t>(tile) * abytes + (qp_pstart(p, b) >> 3)] = static_cast<uint8_t>(a ^ flip);
                });
}

constexpr int QU_NT = 1024;

__global__ __launch_bounds__(QU_NT) void qp_unpermute(const uint16_t* __restrict__ perm,
                                                      const uint8_t* __restrict__ ans,
                                                      const uint16_t* __restrict__ tab, IdsGeom g, uint32_t neg,
                                                      uint32_t* __restrict__ out)
{
    __shared__ alignas(16) uint8_t a[QA_MAX_ABYTES];
    const uint32_t tile = blockIdx.x, t = threadIdx.x;
    const uint64_t base = static_cast<uint64_t>(tile) * TILE;
    const uint32_t abytes = qp_abytes(g.NB);
    // queries of the real buckets sit below the sentinel run's padded start
    const uint32_t in_range =
        qp_pstart(tab[(static_cast<uint64_t>(tile / TB) * (g.NB + 1) + g.NB) * TB + tile % TB], g.NB);
    const uint4* a_src = reinterpret_cast<const uint4*>(ans + static_cast<uint64_t>(tile) * abytes);
    for (uint32_t u = t; u < abytes / 16u; u += QU_NT) reinterpret_cast<uint4*>(a)[u] = ld_stream(a_src + u);
    __syncthreads();
    auto answer = [&](uint32_t pp) { return pp < in_range ? (static_cast<uint32_t>(a[pp >> 3]) >> (pp & 7u)) & 1u : neg; };
    if (base + TILE <= g.n && (reinterpret_cast<uintptr_t>(out) & 15u) == 0) {
        // four queries a thread: 8-byte perm loads, 16-byte answer stores
        const uint2* p2 = reinterpret_cast<const uint2*>(perm + base);
        uint4* o4 = reinterpret_cast<uint4*>(out + base);
#pragma unroll
        for (uint32_t k = 0; k < TILE / (4u * QU_NT); ++k) {
            const uint32_t q = t + k * QU_NT;
            // the permutation is read once, in order: a nontemporal stream
            const uint64_t pp64 = __builtin_nontemporal_load(reinterpret_cast<const uint64_t*>(p2) + q);
            const uint2 pp = make_uint2(static_cast<uint32_t>(pp64), static_cast<uint32_t>(pp64 >> 32));
            st_stream(o4 + q, make_uint4(answer(pp.x & 0xFFFFu), answer(pp.x >> 16), answer(pp.y & 0xFFFFu),
                                         answer(pp.y >> 16)));
        }
    } else {
        for (uint32_t p = t; p < TILE && base + p < g.n; p += QU_NT) out[base + p] = answer(perm[base + p]);
    }
}

int contains_partitioned(const GpuRoaringView& v, const uint32_t* d_ids, uint64_t n, uint32_t* d_out, hipStream_t s)
{
    IdsGeom g{};
    g.n = n;
    g.K = v.key_index ? v.max_key + 1u : 65536u;  // without a key index every key may hold a container
    g.NB = (g.K + BK_KEYS - 1) / BK_KEYS;
    const uint64_t n_tiles = (n + TILE - 1) / TILE;
    if (n_tiles > 0xFFFFFFFFull / TILE_WORDS) {
        set_error("cr_contains_batch: %llu queries exceed the partitioned mode's tile count",
                  static_cast<unsigned long long>(n));
        return CR_ERR_UNSUPPORTED;
    }
    g.n_tiles = static_cast<uint32_t>(n_tiles);
    g.G = std::max<uint32_t>(1, std::min<uint32_t>(num_cus(), (g.n_tiles + TB - 1) / TB));
    g.vec = (reinterpret_cast<uintptr_t>(d_ids) & 15u) == 0;
    Carver c;
    // qp_answer reads up to 5 words past a field group's first: slack past the last tile
    const size_t o_part = c.add(sizeof(uint32_t) * (static_cast<uint64_t>(g.n_tiles) * TILE_WORDS + 8));
    const size_t o_tab = c.add(sizeof(uint16_t) * static_cast<uint64_t>((g.n_tiles + TB - 1) / TB) * TB * (g.NB + 1));
    const size_t o_perm = c.add(sizeof(uint16_t) * static_cast<uint64_t>(g.n_tiles) * TILE);
    const size_t o_ans = c.add(static_cast<uint64_t>(g.n_tiles) * qp_abytes(g.NB));
    const size_t o_gmax = c.add(sizeof(uint32_t) * g.G);
    const size_t o_tot = c.add(sizeof(IdsTotals));
    Scratch sc;
    CR_RET(sc.alloc(c.total, s));
    {
        CR_TIMED("qp_tile_sort", s);
        ids_tile_sort<true><<<g.G, TS_NT, 0, s>>>(d_ids, g, sc.at<uint32_t>(o_part), sc.at<uint16_t>(o_tab),
                                                  sc.at<uint32_t>(o_gmax), sc.at<IdsTotals>(o_tot),
                                                  sc.at<uint16_t>(o_perm), nullptr);
    }
    CR_LAUNCH_CHECK();
    {
        CR_TIMED("qp_answer", s);
        qp_answer<<<build_grid(g.NB), BUILD_NT, 0, s>>>(sc.at<uint32_t>(o_part), sc.at<uint16_t>(o_tab), g, v,
                                                        sc.at<uint8_t>(o_ans));
    }
    CR_LAUNCH_CHECK();
    {
        CR_TIMED("qp_unpermute", s);
        qp_unpermute<<<g.n_tiles, QU_NT, 0, s>>>(sc.at<uint16_t>(o_perm), sc.at<uint8_t>(o_ans),
                                                 sc.at<uint16_t>(o_tab), g, v.negated ? 1u : 0u, d_out);
    }
    CR_LAUNCH_CHECK();
    return CR_OK;
}

}  // namespace crimpl

using namespace crimpl;

extern "C" int cr_contains_batch(const cr_gpu_roaring_view* view, const uint32_t* d_ids, uint64_t n, uint32_t* d_out,
                                 uint32_t mode, cr_stream_t stream)
{
    if (!view || (n && (!d_ids || !d_out)) || mode > CR_QUERY_PARTITIONED) {
        set_error("cr_contains_batch: invalid argument");
        return CR_ERR_INVALID;
    }
    if (n == 0) return CR_OK;
    GpuRoaringView v;
    static_assert(sizeof(v) == sizeof(*view), "view layout");
    std::memcpy(&v, view, sizeof(v));
    // The all-bitmap fast paths read key_index; a view without one takes the
    // general lookup, as contains() does (roaring_view.cuh:45).
    v.all_bitmap = v.all_bitmap && v.key_index != nullptr;
    hipStream_t s = as_stream(stream);
    if (mode == CR_QUERY_PARTITIONED) return contains_partitioned(v, d_ids, n, d_out, s);
    const uint32_t cus = num_cus();
    const uint64_t per_block = static_cast<uint64_t>(Q_NT) * QPT;
    const unsigned grid = static_cast<unsigned>(
        std::max<uint64_t>(1, std::min<uint64_t>((n + per_block - 1) / per_block, static_cast<uint64_t>(cus) * 16u)));
    {
        CR_TIMED("contains", s);
        if (v.all_bitmap && mode == CR_QUERY_CONTAINS) {
            contains_allbitmap<false><<<grid, Q_NT, 0, s>>>(v, d_ids, n, d_out);
        } else if (v.all_bitmap && mode == CR_QUERY_WAVEFRONT) {
            contains_allbitmap<true><<<grid, Q_NT, 0, s>>>(v, d_ids, n, d_out);
        } else if (mode == CR_QUERY_WAVEFRONT) {
            const unsigned gi = static_cast<unsigned>(std::max<uint64_t>(
                1, std::min<uint64_t>((n + Q_NT * QI - 1) / (Q_NT * QI), static_cast<uint64_t>(cus) * 16u)));
            contains_interleaved<<<gi, Q_NT, 0, s>>>(v, d_ids, n, d_out);
        } else if (mode == CR_QUERY_WAVEFRONT_API) {
            contains_general<CR_QUERY_WAVEFRONT><<<grid, Q_NT, 0, s>>>(v, d_ids, n, d_out);
        } else {
            contains_general<CR_QUERY_CONTAINS><<<grid, Q_NT, 0, s>>>(v, d_ids, n, d_out);
        }
    }
    CR_LAUNCH_CHECK();
    return CR_OK;
}

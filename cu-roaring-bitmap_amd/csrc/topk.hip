// Fused filtered brute-force top-k on fp32 MFMA (no reference implementation;
// the reference motivates the path only in prose, README.md:265).
//
// For each query q: the k smallest squared L2 distances ||q - x_i||^2 over the
// base vectors i that pass the filter, ascending, ties broken by the smaller id.
//
//   1. tk_enum_count / tk_enum_write: the passing ids of [0, n_base), in
//      ascending order, via GpuRoaringView::contains (any layout, negated too).
//   2. tk_dist: grid = chunks of the passing ids x blocks of 256 queries.  Each
//      wave keeps 32 queries in registers as the MFMA B operand and streams
//      64-row base tiles through LDS (double buffered, rows gathered by id) as
//      the A operand: d = ||q||^2 + ||x||^2 - 2 q.x with
//      v_mfma_f32_32x32x2f32.  That expansion loses relative precision for
//      near-duplicate vectors, so it only gates: a row that may beat its
//      query's current k-th best gets its fp32 distance sum((q - x)^2)
//      recomputed from the LDS tile, and enters the wave's candidate buffer
//      if it does.  A full buffer is merged into per-(chunk, query) sorted
//      top-k lists; every stored and returned distance is the direct one.
//   3. tk_merge: one wave per query merges its chunk lists into the answer.
// Before tk_dist, tk_pairs and tk_select run on both paths: for a small set
// (at most the small-set limit of passing rows) tk_pairs writes every row's
// distance estimate and tk_select picks each query's k from them, and the list
// path's kernels exit (or are not launched when the host knows the count);
// for a larger set they bound each query's k-th distance from the first rows,
// the bound tk_dist starts from.
#include <algorithm>
#include <atomic>
#include <cstring>

#include "cu_roaring/device/roaring_view.hpp"
#include "image.hpp"
#include "internal.hpp"

namespace crimpl {

using cu_roaring::GpuRoaringView;

namespace {

constexpr uint32_t TK_ENUM_IDS = 8192;  // ids per enumeration workgroup
constexpr int TK_ENUM_NT = 256;
constexpr int TK_NT = 512;  // distance kernel: 8 waves
constexpr int TK_WAVES = TK_NT / 64;
constexpr uint32_t TK_QW = 32;                  // queries per wave (MFMA N)
constexpr uint32_t TK_QB = TK_WAVES * TK_QW;    // queries per workgroup
constexpr int TK_ROWS = 64;                     // base rows per tile (two 32-row MFMA blocks)
constexpr uint32_t TK_CB = 512;                 // candidate buffer entries per wave
constexpr uint32_t TK_KMAX = 256;
constexpr uint32_t TK_NOID = 0xFFFFFFFFu;
constexpr int TK_MERGE_NT = 256;
// Bound on |MFMA-expansion distance - fp32 direct distance| per unit of
// |q|^2 + |x|^2 at dim <= 128: about (2*128 + 4) unit roundoffs for the dot
// product, the two norms and the combination, plus the direct sum's own
// 128-term bound, rounded up.
constexpr float TK_GATE_ERR = 4e-5f;
// The MFMA estimate with the (1 - TK_GATE_ERR) scaling is at most the fp32
// distance; adding TK_SEED_ERR (qg + xg) makes it at least the fp32 distance
// (2 E / (1 - E) with E = TK_GATE_ERR, rounded up for the fp32 arithmetic).
constexpr float TK_SEED_ERR = 3.0f * TK_GATE_ERR;

typedef float f32x16 __attribute__((ext_vector_type(16)));

// Order-preserving map of fp32 values to u32 (and back).
__device__ __forceinline__ uint32_t tk_ordered(float f)
{
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float tk_unordered(uint32_t u)
{
    return __uint_as_float((u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u);
}

// Upper bound of a row's fp32 distance from its estimate (a lower bound) and
// the scaled norms; one fused operation, so every kernel computes the same value.
__device__ __forceinline__ float tk_upper(float est, float qg, float xg) { return __fmaf_rn(TK_SEED_ERR, qg + xg, est); }

// Strict order of (distance, id) pairs: the output order.
__device__ __forceinline__ bool tk_less(float ad, uint32_t ai, float bd, uint32_t bi)
{
    return ad < bd || (ad == bd && ai < bi);
}

// Number of entries of the sorted list (d, id)[0, n) that order before (yd, yi).
__device__ __forceinline__ uint32_t tk_lower_bound(const float* d, const uint32_t* id, uint32_t n, float yd,
                                                   uint32_t yi)
{
    uint32_t lo = 0, hi = n;
    while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (tk_less(d[mid], id[mid], yd, yi))
            lo = mid + 1;
        else
            hi = mid;
    }
    return lo;
}

__device__ __forceinline__ uint64_t lanemask_lt() { return (1ull << __lane_id()) - 1ull; }

struct TkArgs {
    const float* base;
    const float* queries;
    const uint32_t* sel;    // passing ids ascending (nullptr: every id of [0, n_base))
    const uint32_t* n_sel;  // device count of sel
    uint64_t n_base;
    uint32_t n_q;
    uint32_t dim;
    uint32_t k;
    uint32_t n_chunks;  // multiple of 8
    uint32_t vec;       // rows are 16-B aligned with dim % 4 == 0
    uint32_t qvec;      // so are the queries
    float* list_d;      // two planes of [n_chunks][n_q][k]: a merge reads one, writes the other
    uint32_t* list_id;  // the same two planes
    size_t plane;       // elements per plane
    uint32_t* list_n;   // [n_chunks][n_q]: list length | (plane holding the list << 31)
    uint32_t* tau;      // [n_q] bits of the smallest k-th distance any chunk has reached
    uint32_t* tau_m;    // [n_chunks][n_q] bits of each chunk's m_rank-th distance (+inf: fewer entries)
    uint32_t m_rank;    // ceil(2k / n_chunks)
    // Small sets: with at most small_max rows the distance kernel writes every
    // estimate (pd[q][row], lower bounds of the fp32 distances) with the scaled
    // norms (pq[q], px[row]), and tk_select picks each query's k from them.
    uint32_t small_max;  // 0: never
    float* pd;           // [n_qb * TK_QB][small_max] (rows past n_q unused)
    float* pq;           // [n_q]
    float* px;           // [small_max]
    uint32_t* qlo;       // [n_q] order-preserving bits of the smallest upper bound of the query's rows
    uint32_t* qhi;       // [n_q] ... and of the largest
    // The host knew the passing count to be within small_max (no filter and a
    // small base, or a filter's recorded cardinality) and launched no list
    // path; tk_select then answers any count (every row a candidate past it).
    uint32_t list_off;
};

// Rows the distance kernel covers, and whether the small-set path takes them.
__device__ __forceinline__ uint64_t tk_rows(const TkArgs& a) { return a.sel ? static_cast<uint64_t>(*a.n_sel) : a.n_base; }
__device__ __forceinline__ bool tk_small(const TkArgs& a, uint64_t n_rows)
{
    return a.small_max != 0 && n_rows <= a.small_max;
}
// Larger sets: the small-set kernels first bound each query's k-th distance
// from the upper bounds of the first rows (at most small_max of them), and the
// list path starts from that bound instead of from +inf.
constexpr uint32_t TK_SEED_ROWS = 16384;
constexpr uint32_t TK_SEED_ROWS_PER_K = 256;
__device__ __forceinline__ uint32_t tk_seed_rows(const TkArgs& a, uint64_t n_rows)
{
    if (a.small_max == 0 || tk_small(a, n_rows)) return 0;
    const uint64_t want = std::max<uint64_t>(TK_SEED_ROWS, static_cast<uint64_t>(TK_SEED_ROWS_PER_K) * a.k);
    return static_cast<uint32_t>(std::min<uint64_t>(std::min<uint64_t>(n_rows, a.small_max), want));
}

// The call's state: every query's bound (tau) and each chunk's m_rank-th
// distance (tau_m) at +inf, and for the small-set path the range of the upper
// bounds (qlo at the largest value, qhi at the smallest); thread i of `stride`.
__device__ __forceinline__ void tk_init_from(const TkArgs& a, uint64_t i, uint64_t stride)
{
    const uint64_t n = std::max<uint64_t>(static_cast<uint64_t>(a.n_chunks) * a.n_q, a.n_q);
    for (; i < n; i += stride) {
        if (i < static_cast<uint64_t>(a.n_chunks) * a.n_q) a.tau_m[i] = 0x7F800000u;
        if (i < a.n_q) {
            a.tau[i] = 0x7F800000u;
            if (a.small_max) {
                a.qlo[i] = 0xFFFFFFFFu;
                a.qhi[i] = 0u;
            }
        }
    }
}

// ---- 1. passing ids ---------------------------------------------------------

// A workgroup covers 8192 consecutive ids, a 256-word slice of one key's
// container: the container is looked up once, and thread t takes word t of the
// slice -- from the bitmap, or from the container's image built in LDS for an
// array or run container -- complemented for a negated filter (contains()
// answers `negated` for absent keys) and cut at n_base.
static_assert(TK_ENUM_IDS == 32u * TK_ENUM_NT && 65536u % TK_ENUM_IDS == 0, "one word per thread, one key per block");

__device__ uint32_t tk_enum_word(const GpuRoaringView& v, uint64_t n_base, uint32_t* img, int32_t* cover, int32_t* s_c)
{
    const uint32_t t = threadIdx.x;
    const uint64_t base = static_cast<uint64_t>(blockIdx.x) * TK_ENUM_IDS;
    const uint32_t key = static_cast<uint32_t>(base >> 16);
    if (v.key_index && key <= v.max_key) {
        if (t == 0) {
            const uint16_t e = v.key_index[key];
            *s_c = e == 0xFFFFu ? -1 : static_cast<int32_t>(e);
        }
    } else if (key > v.max_key && v.key_index) {
        if (t == 0) *s_c = -1;
    } else if (t < 64) {
        const uint32_t pos = wave_lower_bound_u16(v.keys, v.n_containers, key);
        if (t == 0) *s_c = (pos < v.n_containers && v.keys[pos] == key) ? static_cast<int32_t>(pos) : -1;
    }
    __syncthreads();
    const int32_t c = *s_c;
    const uint32_t w0 = static_cast<uint32_t>(base & 0xFFFFu) >> 5;  // first word of the slice in the container
    uint32_t word = 0;
    const uint8_t type = c >= 0 ? static_cast<uint8_t>(v.types[c]) : uint8_t(0xFF);  // block-uniform
    if (type == CR_BITMAP) {
        word = reinterpret_cast<const uint32_t*>(v.bitmap_data + v.offsets[c] / 8u)[w0 + t];
    } else if (type == CR_ARRAY || type == CR_RUN) {
        expand_img<TK_ENUM_NT>(type, (type == CR_ARRAY ? v.array_data : v.run_data) + v.offsets[c] / 2u,
                               v.cardinalities[c], img, cover);
        word = img[w0 + t];
    }
    if (v.negated) word = ~word;
    const uint64_t id0 = base + 32u * t;
    if (id0 >= n_base) word = 0;
    else if (n_base - id0 < 32u) word &= (1u << (n_base - id0)) - 1u;
    return word;
}

// Also initialises the call's state (tk_init_from), which saves a launch.
__global__ __launch_bounds__(TK_ENUM_NT) void tk_enum_count(GpuRoaringView v, uint64_t n_base, uint32_t* counts,
                                                            TkArgs a)
{
    tk_init_from(a, static_cast<uint64_t>(blockIdx.x) * TK_ENUM_NT + threadIdx.x,
                 static_cast<uint64_t>(gridDim.x) * TK_ENUM_NT);
    __shared__ alignas(16) uint32_t img[2048];
    __shared__ int32_t cover[2048];
    __shared__ int32_t s_c;
    __shared__ uint32_t red[TK_ENUM_NT / 64];
    const uint32_t c = block_sum<TK_ENUM_NT>(__popc(tk_enum_word(v, n_base, img, cover, &s_c)), red);
    if (threadIdx.x == 0) counts[blockIdx.x] = c;
}

__global__ __launch_bounds__(TK_ENUM_NT) void tk_enum_write(GpuRoaringView v, uint64_t n_base, const uint32_t* counts,
                                                            uint32_t* sel, uint32_t* n_sel)
{
    __shared__ alignas(16) uint32_t img[2048];
    __shared__ int32_t cover[2048];
    __shared__ int32_t s_c;
    __shared__ uint32_t red[TK_ENUM_NT / 64];
    uint32_t pre = 0;
    for (uint32_t i = threadIdx.x; i < blockIdx.x; i += TK_ENUM_NT) pre += counts[i];
    const uint32_t run = block_sum<TK_ENUM_NT>(pre, red);
    const uint32_t word = tk_enum_word(v, n_base, img, cover, &s_c);
    uint32_t tot;
    uint32_t pos = run + block_excl_scan<TK_ENUM_NT>(__popc(word), red, tot);
    const uint32_t id0 = static_cast<uint32_t>(static_cast<uint64_t>(blockIdx.x) * TK_ENUM_IDS) + 32u * threadIdx.x;
    for (uint32_t x = word; x; x &= x - 1) sel[pos++] = id0 + static_cast<uint32_t>(__builtin_ctz(x));
    if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) *n_sel = run + tot;
}

// ---- 2. distances and per-chunk selection ----------------------------------

// Per-wave selection state in LDS.
struct TkWave {
    float cd[TK_CB];  // candidate buffer: distance, id, query slot (0..31)
    uint32_t cid[TK_CB];
    uint64_t sk[TK_CB];  // sort keys during a merge: query << 32 | distance bits
    float td[TK_QW];     // the query's k-th best so far (+inf, NOID while the list is short)
    float tm[TK_QW];     // the query's m_rank-th best so far (+inf while the list is shorter)
    uint32_t tid[TK_QW];
    uint32_t ln[TK_QW];   // list length
    uint32_t par[TK_QW];  // plane holding the list
    uint32_t qcnt[TK_QW];
    uint32_t qoff[TK_QW];
    uint8_t cq[TK_CB];
};

template <int DP>
struct TkLds {
    float tile[2][TK_ROWS * (DP + 4)];  // rows skewed by 16 B: conflict-free b128 reads
    float xg[2][TK_ROWS];               // (1 - TK_GATE_ERR) |x|^2, NaN for rows past the chunk
    uint32_t id[2][TK_ROWS];
    TkWave w[TK_WAVES];
    uint32_t flush_req;  // tile index at which some wave asked every wave to merge
};

__device__ __forceinline__ float tk_atomic_load(const uint32_t* p)
{
    return __uint_as_float(__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// Bound on the query's k-th distance from the chunks' m_rank-th distances: the
// chunks that have published one hold at least m_rank rows each at or below
// the largest of them, so once they number k / m_rank or more, that largest
// value bounds the k-th distance of the union.  The lane pair of the query
// (j, j + 32) splits the chunks between its two lanes.
__device__ __forceinline__ float tk_spread_bound(const uint32_t* tau_m, uint32_t n_chunks, uint32_t n_q, uint32_t q,
                                                 bool qok, uint32_t h, uint32_t k, uint32_t m_rank)
{
    float mx = 0.f;
    uint32_t c_fin = 0;
    if (qok) {
        for (uint32_t c = h; c < n_chunks; c += 2) {
            const float v = tk_atomic_load(tau_m + static_cast<size_t>(c) * n_q + q);
            if (v != __builtin_inff()) {
                ++c_fin;
                mx = fmaxf(mx, v);
            }
        }
    }
    c_fin += __shfl_xor(c_fin, 32, 64);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    return c_fin * m_rank >= k ? mx : __builtin_inff();
}

// Merges the wave's candidate buffer into the sorted top-k lists of its
// queries (global memory, [chunk][query][k] in two planes) and publishes every
// full list's k-th distance to the shared per-query bound.  Wave-level: no
// block barrier.  The whole buffer is sorted by (query, distance, id) in one
// bitonic network, which leaves each query's candidates as a sorted run; then
// the lane of each query walks its list (read from its current plane) and
// its run together and writes the first min(k, n + nc) of the union to the
// other plane.  Distances are non-negative, so their bits order as values.
__device__ __forceinline__ void tk_flush(TkWave& W, uint32_t cnt, uint32_t k, uint32_t m_rank, uint32_t nq_wave,
                                         float* gd_row, uint32_t* gi_row, size_t plane, uint32_t* tau_q0,
                                         uint32_t* tau_m_q0)
{
    const uint32_t lane = __lane_id();
    if (lane < TK_QW) W.qcnt[lane] = 0;
    __builtin_amdgcn_wave_barrier();
    for (uint32_t e = lane; e < cnt; e += 64) atomicAdd(&W.qcnt[W.cq[e]], 1u);
    uint32_t P = 64;
    while (P < cnt) P <<= 1;
    for (uint32_t e = lane; e < P; e += 64) {
        if (e < cnt) {
            W.sk[e] = (static_cast<uint64_t>(W.cq[e]) << 32) | __float_as_uint(W.cd[e]);
        } else {
            W.sk[e] = ~0ull;
            W.cid[e] = TK_NOID;
        }
    }
    __builtin_amdgcn_wave_barrier();
    const uint32_t c_l = lane < TK_QW ? W.qcnt[lane] : 0u;
    const uint32_t o_l = wave_incl_scan(c_l) - c_l;
    for (uint32_t size = 2; size <= P; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t pp = lane; pp < P / 2; pp += 64) {
                const uint32_t i = 2 * stride * (pp / stride) + (pp % stride);
                const uint32_t i2 = i + stride;
                const uint64_t a0 = W.sk[i], a1 = W.sk[i2];
                const uint32_t b0 = W.cid[i], b1 = W.cid[i2];
                const bool up = (i & size) == 0;
                const bool lt = a1 < a0 || (a1 == a0 && b1 < b0);
                if (lt == up) {
                    W.sk[i] = a1;
                    W.cid[i] = b1;
                    W.sk[i2] = a0;
                    W.cid[i2] = b0;
                }
            }
            __builtin_amdgcn_wave_barrier();
        }
    }
    if (lane < nq_wave && c_l > 0) {
        const uint32_t n = W.ln[lane], par = W.par[lane];
        const float* ind = gd_row + par * plane + static_cast<size_t>(lane) * k;
        const uint32_t* ini = gi_row + par * plane + static_cast<size_t>(lane) * k;
        float* outd = gd_row + (par ^ 1u) * plane + static_cast<size_t>(lane) * k;
        uint32_t* outi = gi_row + (par ^ 1u) * plane + static_cast<size_t>(lane) * k;
        const uint32_t m = min(k, n + c_l);
        uint32_t ia = 0, ib = o_l;
        const uint32_t eb = o_l + c_l;
        float xa = n ? ind[0] : __builtin_inff();
        uint32_t xia = n ? ini[0] : TK_NOID;
        float yb = __uint_as_float(static_cast<uint32_t>(W.sk[ib]));
        uint32_t yib = W.cid[ib];
        float td = W.td[lane], tm = W.tm[lane];
        uint32_t tid = W.tid[lane];
        for (uint32_t r = 0; r < m; ++r) {
            const bool take_a = ia < n && (ib >= eb || tk_less(xa, xia, yb, yib));
            float d;
            uint32_t id;
            if (take_a) {
                d = xa;
                id = xia;
                if (++ia < n) {
                    xa = ind[ia];
                    xia = ini[ia];
                }
            } else {
                d = yb;
                id = yib;
                if (++ib < eb) {
                    yb = __uint_as_float(static_cast<uint32_t>(W.sk[ib]));
                    yib = W.cid[ib];
                }
            }
            outd[r] = d;
            outi[r] = id;
            if (r == k - 1) {
                td = d;
                tid = id;
            }
            if (r == m_rank - 1) tm = d;
        }
        W.td[lane] = td;
        W.tid[lane] = tid;
        W.tm[lane] = tm;
        W.ln[lane] = m;
        W.par[lane] = par ^ 1u;
    }
    __builtin_amdgcn_wave_barrier();
    if (lane < nq_wave) {
        if (W.ln[lane] == k) atomicMin(tau_q0 + lane, __float_as_uint(W.td[lane]));
        if (W.ln[lane] >= m_rank)
            __hip_atomic_store(tau_m_q0 + lane, __float_as_uint(W.tm[lane]), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    // The lists are re-read by this wave at its next merge.
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
}

template <int DP>
__device__ __forceinline__ void tk_load_rows(const TkArgs& a, uint64_t row0, uint64_t row_end, float4 (&pre)[DP / 32],
                                             uint32_t (&pid)[DP / 32])
{
    constexpr int TPR = DP / 4;            // threads per row (one float4 each)
    constexpr int RPP = TK_NT / TPR;       // rows per pass
    const uint32_t t = threadIdx.x;
    const uint32_t c = (t % TPR) * 4;      // first column of this thread
#pragma unroll
    for (int p = 0; p < DP / 32; ++p) {
        const uint64_t r = row0 + static_cast<uint64_t>(p * RPP + t / TPR);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        uint32_t id = TK_NOID;
        if (r < row_end) {
            id = a.sel ? a.sel[r] : static_cast<uint32_t>(r);
            const float* src = a.base + static_cast<size_t>(id) * a.dim;
            if (a.vec) {
                if (c < a.dim) v = *reinterpret_cast<const float4*>(src + c);
            } else {
                if (c + 0 < a.dim) v.x = src[c + 0];
                if (c + 1 < a.dim) v.y = src[c + 1];
                if (c + 2 < a.dim) v.z = src[c + 2];
                if (c + 3 < a.dim) v.w = src[c + 3];
            }
        }
        pre[p] = v;
        pid[p] = id;
    }
}

// The prefetch of a persistent loop, without branches or selects on loaded
// values (either makes the compiler wait for the loads where they are issued):
// the raw ids of a tile's rows, sel[min(r, last)] (or r without a filter),
// loaded a tile ahead of their use; tk_ids_valid then marks the rows past the
// tile as TK_NOID, and tk_load_rows_nb loads a row for every id (row 0 stands
// in for TK_NOID; tk_store_rows stores zeros for it).
template <int DP, bool SEL>
__device__ __forceinline__ void tk_ids_raw(const TkArgs& a, uint64_t row0, uint64_t last, uint32_t (&raw)[DP / 32])
{
    constexpr int TPR = DP / 4;
    constexpr int RPP = TK_NT / TPR;
#pragma unroll
    for (int p = 0; p < DP / 32; ++p) {
        const uint64_t r = row0 + static_cast<uint64_t>(p * RPP + threadIdx.x / TPR);
        raw[p] = SEL ? a.sel[std::min<uint64_t>(r, last)] : static_cast<uint32_t>(r);
    }
}

template <int DP>
__device__ __forceinline__ void tk_ids_valid(uint64_t row0, uint64_t row_end, uint32_t (&pid)[DP / 32])
{
    constexpr int TPR = DP / 4;
    constexpr int RPP = TK_NT / TPR;
#pragma unroll
    for (int p = 0; p < DP / 32; ++p) {
        const uint64_t r = row0 + static_cast<uint64_t>(p * RPP + threadIdx.x / TPR);
        if (r >= row_end) pid[p] = TK_NOID;
    }
}

template <int DP>
__device__ __forceinline__ void tk_load_rows_nb(const TkArgs& a, const uint32_t (&pid)[DP / 32], float4 (&pre)[DP / 32])
{
    constexpr int TPR = DP / 4;
    const uint32_t c = (threadIdx.x % TPR) * 4;
#pragma unroll
    for (int p = 0; p < DP / 32; ++p) {
        const uint32_t id = pid[p] != TK_NOID ? pid[p] : 0u;
        const float* src = a.base + static_cast<size_t>(id) * a.dim;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (a.vec) {
            if (c < a.dim) v = *reinterpret_cast<const float4*>(src + c);
        } else {
            if (c + 0 < a.dim) v.x = src[c + 0];
            if (c + 1 < a.dim) v.y = src[c + 1];
            if (c + 2 < a.dim) v.z = src[c + 2];
            if (c + 3 < a.dim) v.w = src[c + 3];
        }
        pre[p] = v;
    }
}

// Sum over aligned groups of W lanes (8, 16 or 32) with DPP moves, no LDS
// round trips: quad swaps, the half-row and row mirrors, then (W = 32) row
// 15's value broadcast into the next row.  Every lane of a group holds the
// total for W <= 16, the group's upper 16 lanes for W = 32.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float tk_dpp(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}

template <int W>
__device__ __forceinline__ float tk_group_sum(float x)
{
    static_assert(W == 8 || W == 16 || W == 32, "lane groups of 8, 16 or 32");
    x += tk_dpp<0xB1, 0xF>(x);   // quad_perm [1, 0, 3, 2]
    x += tk_dpp<0x4E, 0xF>(x);   // quad_perm [2, 3, 0, 1]
    x += tk_dpp<0x141, 0xF>(x);  // row_half_mirror
    if constexpr (W >= 16) x += tk_dpp<0x140, 0xF>(x);  // row_mirror
    if constexpr (W == 32) x += tk_dpp<0x142, 0xA>(x);  // row_bcast:15 into rows 1 and 3 (rows 0 and 2 add 0)
    return x;
}

template <int DP, class Lds>
__device__ __forceinline__ void tk_store_rows(Lds& L, int buf, const float4 (&pre)[DP / 32],
                                              const uint32_t (&pid)[DP / 32])
{
    constexpr int TPR = DP / 4;
    constexpr int RPP = TK_NT / TPR;
    const uint32_t t = threadIdx.x;
#pragma unroll
    for (int p = 0; p < DP / 32; ++p) {
        const int row = p * RPP + static_cast<int>(t / TPR);
        const int c = static_cast<int>(t % TPR) * 4;
        const float4 v = pid[p] != TK_NOID ? pre[p] : make_float4(0.f, 0.f, 0.f, 0.f);
        *reinterpret_cast<float4*>(&L.tile[buf][row * (DP + 4) + c]) = v;
        const float ss = tk_group_sum<TPR>(v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w);
        if (static_cast<int>(t % TPR) == (TPR == 32 ? TPR - 1 : 0)) {  // a lane holding the row's total
            L.xg[buf][row] = pid[p] != TK_NOID ? (1.f - TK_GATE_ERR) * ss : __builtin_nanf("");
            L.id[buf][row] = pid[p];
        }
    }
}

// This lane's query dimensions [h DP/2, h DP/2 + DP/2) into qreg (zeros past
// dim or for a lane without a query): 16-byte loads when the queries allow
// them, each a contiguous 16 bytes of the lane's row, else one float at a
// time.  Returns the sum of their squares.
template <int DP>
__device__ __forceinline__ float tk_load_query(const TkArgs& a, bool qok, uint32_t q, uint32_t h, float (&qreg)[DP / 2])
{
    const float* src = a.queries + static_cast<size_t>(q) * a.dim + h * (DP / 2);
    if (a.qvec) {
#pragma unroll
        for (int s = 0; s < DP / 2; s += 4) {
            const uint32_t c = h * (DP / 2) + s;
            const float4 v = (qok && c < a.dim) ? *reinterpret_cast<const float4*>(src + s) : make_float4(0.f, 0.f, 0.f, 0.f);
            qreg[s] = v.x, qreg[s + 1] = v.y, qreg[s + 2] = v.z, qreg[s + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int s = 0; s < DP / 2; ++s) {
            const uint32_t c = h * (DP / 2) + s;
            qreg[s] = (qok && c < a.dim) ? src[s] : 0.f;
        }
    }
    float part = 0.f;
#pragma unroll
    for (int s = 0; s < DP / 2; ++s) part += qreg[s] * qreg[s];
    return part;
}

// Base row held by accumulator register rr (0..31: block rr/16, register
// rr%16) of the lane half hh.
__device__ __forceinline__ int tk_row(int rr, int hh)
{
    return (rr >> 4) * 32 + 8 * ((rr & 15) >> 2) + 4 * hh + (rr & 3);
}

template <int DP, bool SEL>
__global__ __launch_bounds__(TK_NT) void tk_dist(TkArgs a)
{
    __shared__ TkLds<DP> L;
    const uint32_t lane = __lane_id();
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t h = lane >> 5;    // lane half: which half of the dimensions it feeds
    const uint32_t j = lane & 31u;   // query column of this lane
    TkWave& W = L.w[wave];

    // Blocks are dispatched round-robin over the 8 XCDs: the blocks of one XCD
    // take consecutive query blocks of the same chunks, so they share the
    // chunk's base rows in that XCD's L2.
    const uint32_t n_qb = (a.n_q + TK_QB - 1) / TK_QB;
    const uint32_t per_xcd = gridDim.x / 8;
    const uint32_t pidx = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    const uint32_t chunk = pidx / n_qb;
    const uint32_t qb = pidx % n_qb;

    const uint64_t n_rows = tk_rows(a);
    if (tk_small(a, n_rows)) return;  // tk_pairs and tk_select answer small sets
    const uint64_t rpc = ((n_rows + a.n_chunks - 1) / a.n_chunks + TK_ROWS - 1) / TK_ROWS * TK_ROWS;
    const uint64_t r0 = std::min<uint64_t>(n_rows, static_cast<uint64_t>(chunk) * rpc);
    const uint64_t r1 = std::min<uint64_t>(n_rows, r0 + rpc);
    const uint32_t n_tiles = static_cast<uint32_t>((r1 - r0 + TK_ROWS - 1) / TK_ROWS);

    const uint32_t q0 = qb * TK_QB + wave * TK_QW;
    const uint32_t nq_wave = q0 < a.n_q ? std::min<uint32_t>(TK_QW, a.n_q - q0) : 0u;
    const bool qok = j < nq_wave;
    const size_t list_row = (static_cast<size_t>(chunk) * a.n_q + q0) * a.k;
    uint32_t* tau_q0 = a.tau + q0;
    uint32_t* tau_m_q0 = a.tau_m + static_cast<size_t>(chunk) * a.n_q + q0;

    if (lane < TK_QW) {
        W.td[lane] = __builtin_inff();
        W.tm[lane] = __builtin_inff();
        W.tid[lane] = TK_NOID;
        W.ln[lane] = 0;
        W.par[lane] = 0;
    }
    if (threadIdx.x == 0) L.flush_req = TK_NOID;

    // B operand: this lane's query, dimensions [h*DP/2, h*DP/2 + DP/2).
    float qreg[DP / 2];
    const float qpart = tk_load_query<DP>(a, qok, q0 + j, h, qreg);
    const float qg = (1.f - TK_GATE_ERR) * (qpart + __shfl_xor(qpart, 32, 64));

    // The prefetch as in tk_pairs: tile t + 1's rows (ids known since tile
    // t - 1) and tile t + 2's raw ids are issued before tile t's MFMA and
    // waited for after it.
    auto tile_r0 = [&](uint32_t i) { return r0 + static_cast<uint64_t>(i) * TK_ROWS; };
    auto tile_r1 = [&](uint32_t i) { return std::min<uint64_t>(r1, tile_r0(i) + TK_ROWS); };
    const uint64_t last = n_rows > 0 ? n_rows - 1 : 0;
    float4 pre[DP / 32];
    uint32_t pid[DP / 32], nid[DP / 32];
    if constexpr (SEL) {
        if (n_rows > 0) tk_ids_raw<DP, SEL>(a, tile_r0(1), last, nid);
    }
    if (n_tiles > 0) {
        tk_load_rows<DP>(a, r0, r1, pre, pid);
        tk_store_rows<DP>(L, 0, pre, pid);
    }
    if constexpr (SEL) {
#pragma unroll
        for (int p = 0; p < DP / 32; ++p) pid[p] = n_rows > 0 ? nid[p] : TK_NOID;
        tk_ids_valid<DP>(tile_r0(1), tile_r1(1), pid);
    }
    __syncthreads();

    // Thresholds of this lane's query: the own list's k-th best (td, tidv) and
    // the bound shared by all chunks (tsh).  A row whose distance exceeds
    // either cannot be in the answer.
    float td = __builtin_inff();
    uint32_t tidv = TK_NOID;
    float tsh = __builtin_inff();
    float seed = __builtin_inff();  // bound on the chunk's k-th best from its first tile
    uint32_t cnt = 0;  // wave-uniform fill of the candidate buffer
    for (uint32_t t = 0; t < n_tiles; ++t) {
        const int b = static_cast<int>(t & 1u);
        if constexpr (SEL) {
            tk_load_rows_nb<DP>(a, pid, pre);
            tk_ids_raw<DP, SEL>(a, tile_r0(t + 2), last, nid);
        } else if (t + 1 < n_tiles) {  // the row numbers are the ids
            tk_load_rows<DP>(a, tile_r0(t + 1), r1, pre, pid);
        }
        const float tsh_new = qok ? tk_atomic_load(tau_q0 + j) : __builtin_inff();

        if (nq_wave > 0) {
            f32x16 acc0 = {}, acc1 = {};
            const float* A0 = &L.tile[b][j * (DP + 4) + h * (DP / 2)];
            const float* A1 = A0 + 32 * (DP + 4);
#pragma unroll
            for (int s = 0; s < DP / 2; s += 4) {
                const float4 x0 = *reinterpret_cast<const float4*>(A0 + s);
                const float4 x1 = *reinterpret_cast<const float4*>(A1 + s);
                acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0.x, qreg[s + 0], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1.x, qreg[s + 0], acc1, 0, 0, 0);
                acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0.y, qreg[s + 1], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1.y, qreg[s + 1], acc1, 0, 0, 0);
                acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0.z, qreg[s + 2], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1.z, qreg[s + 2], acc1, 0, 0, 0);
                acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0.w, qreg[s + 3], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1.w, qreg[s + 3], acc1, 0, 0, 0);
            }
            tsh = fminf(tsh, tsh_new);
            // Gate: the MFMA distance |q|^2 + |x|^2 - 2 q.x lies within
            // TK_GATE_ERR (|q|^2 + |x|^2) of the fp32 direct distance, so a
            // row passes when that margin could put it at or below the
            // thresholds.  Accumulator register r of block u holds base row
            // tk_row(16u + r, h) against query column j.
            // The accumulators become the estimates |q|^2 + |x|^2 - 2 q.x
            // (scaled as above; NaN for rows past the chunk).
#pragma unroll
            for (int rq = 0; rq < 4; ++rq) {
                const float4 g0 = *reinterpret_cast<const float4*>(&L.xg[b][8 * rq + 4 * h]);
                const float4 g1 = *reinterpret_cast<const float4*>(&L.xg[b][32 + 8 * rq + 4 * h]);
                acc0[4 * rq + 0] = qg + g0.x - 2.f * acc0[4 * rq + 0];
                acc0[4 * rq + 1] = qg + g0.y - 2.f * acc0[4 * rq + 1];
                acc0[4 * rq + 2] = qg + g0.z - 2.f * acc0[4 * rq + 2];
                acc0[4 * rq + 3] = qg + g0.w - 2.f * acc0[4 * rq + 3];
                acc1[4 * rq + 0] = qg + g1.x - 2.f * acc1[4 * rq + 0];
                acc1[4 * rq + 1] = qg + g1.y - 2.f * acc1[4 * rq + 1];
                acc1[4 * rq + 2] = qg + g1.z - 2.f * acc1[4 * rq + 2];
                acc1[4 * rq + 3] = qg + g1.w - 2.f * acc1[4 * rq + 3];
            }
            if (t == 0 && a.k <= TK_ROWS) {
                // Seed: the k-th smallest estimate of the first tile's rows
                // (bisection on the lane pair's 64 estimates), raised to an
                // upper estimate, bounds the chunk's k-th best distance, so
                // the first tile yields about k candidates per query instead
                // of all of its rows.
                float lo = __builtin_inff(), hi = -__builtin_inff();
                uint32_t nv = 0;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float e0 = acc0[r], e1 = acc1[r];
                    if (e0 == e0) {
                        lo = fminf(lo, e0);
                        hi = fmaxf(hi, e0);
                        ++nv;
                    }
                    if (e1 == e1) {
                        lo = fminf(lo, e1);
                        hi = fmaxf(hi, e1);
                        ++nv;
                    }
                }
                lo = fminf(lo, __shfl_xor(lo, 32, 64));
                hi = fmaxf(hi, __shfl_xor(hi, 32, 64));
                nv += __shfl_xor(nv, 32, 64);
                float xgmax = L.xg[b][lane];
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) xgmax = fmaxf(xgmax, __shfl_xor(xgmax, o, 64));
                const bool do_seed = qok && nv >= a.k;
                for (int it = 0; it < 24; ++it) {  // invariant: at least k estimates <= hi
                    const float mid = 0.5f * (lo + hi);
                    uint32_t c = 0;
#pragma unroll
                    for (int r = 0; r < 16; ++r) c += (acc0[r] <= mid ? 1u : 0u) + (acc1[r] <= mid ? 1u : 0u);
                    c += __shfl_xor(c, 32, 64);
                    if (c >= a.k)
                        hi = mid;
                    else
                        lo = mid;
                }
                if (do_seed) seed = hi + TK_SEED_ERR * (qg + xgmax);
            }
            const float tgate = fminf(fminf(td, tsh), seed);
            uint32_t pm = 0;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                pm |= (acc0[r] <= tgate ? 1u : 0u) << r;
                pm |= (acc1[r] <= tgate ? 1u : 0u) << (16 + r);
            }
            if (!qok) pm = 0;
            if (__ballot(pm != 0)) {
                // Both lanes of a query (j and j + 32) walk the query's gated
                // rows in the same order; each sums its half of the dimensions
                // and the pair adds the halves.
                uint32_t m0 = __shfl(pm, static_cast<int>(j), 64);
                uint32_t m1 = __shfl(pm, static_cast<int>(j + 32), 64);
                while (__ballot((m0 | m1) != 0)) {
                    if (cnt + TK_QW > TK_CB) {
                        tk_flush(W, cnt, a.k, a.m_rank, nq_wave, a.list_d + list_row, a.list_id + list_row, a.plane, tau_q0, tau_m_q0);
                        cnt = 0;
                        td = W.td[j];
                        tidv = W.tid[j];
                        if (qok) tsh = fminf(tsh, tk_atomic_load(tau_q0 + j));
                        tsh = fminf(tsh, tk_spread_bound(a.tau_m, a.n_chunks, a.n_q, q0 + j, qok, h, a.k, a.m_rank));
                    }
                    int row = -1;
                    if (m0) {
                        row = tk_row(__builtin_ctz(m0), 0);
                        m0 &= m0 - 1;
                    } else if (m1) {
                        row = tk_row(__builtin_ctz(m1), 1);
                        m1 &= m1 - 1;
                    }
                    float e2 = 0.f;
                    if (row >= 0) {
                        const float* xr = &L.tile[b][row * (DP + 4) + h * (DP / 2)];
#pragma unroll
                        for (int s2 = 0; s2 < DP / 2; s2 += 4) {
                            const float4 v = *reinterpret_cast<const float4*>(xr + s2);
                            float e;
                            e = qreg[s2 + 0] - v.x; e2 = fmaf(e, e, e2);
                            e = qreg[s2 + 1] - v.y; e2 = fmaf(e, e, e2);
                            e = qreg[s2 + 2] - v.z; e2 = fmaf(e, e, e2);
                            e = qreg[s2 + 3] - v.w; e2 = fmaf(e, e, e2);
                        }
                    }
                    const float d = e2 + __shfl_xor(e2, 32, 64);
                    bool f = false;
                    uint32_t id = 0;
                    if (h == 0 && row >= 0) {
                        id = L.id[b][row];
                        f = tk_less(d, id, td, tidv) && d <= tsh && d <= seed;
                    }
                    const uint64_t m = __ballot(f);
                    if (f) {
                        const uint32_t pos = cnt + static_cast<uint32_t>(__popcll(m & lanemask_lt()));
                        W.cd[pos] = d;
                        W.cid[pos] = id;
                        W.cq[pos] = static_cast<uint8_t>(j);
                    }
                    cnt += static_cast<uint32_t>(__popcll(m));
                }
            }
        }
        // Merges are taken together: a wave whose buffer is half full asks
        // every wave to merge after the barrier, so the waves of the block
        // stall for one merge at a time rather than one after another.
        if (cnt > TK_CB * 3 / 4 && lane == 0) L.flush_req = t;
        if constexpr (SEL) {
            tk_store_rows<DP>(L, b ^ 1, pre, pid);
#pragma unroll
            for (int p = 0; p < DP / 32; ++p) pid[p] = nid[p];
            tk_ids_valid<DP>(tile_r0(t + 2), tile_r1(t + 2), pid);
        } else if (t + 1 < n_tiles) {
            tk_store_rows<DP>(L, b ^ 1, pre, pid);
        }
        __syncthreads();
        if (L.flush_req == t && cnt > 0) {
            tk_flush(W, cnt, a.k, a.m_rank, nq_wave, a.list_d + list_row, a.list_id + list_row, a.plane, tau_q0, tau_m_q0);
            cnt = 0;
            td = W.td[j];
            tidv = W.tid[j];
            if (qok) tsh = fminf(tsh, tk_atomic_load(tau_q0 + j));
        }
        if (nq_wave > 0 && (t & 7u) == 7u)
            tsh = fminf(tsh, tk_spread_bound(a.tau_m, a.n_chunks, a.n_q, q0 + j, qok, h, a.k, a.m_rank));
    }
    if (nq_wave > 0) {
        if (cnt) tk_flush(W, cnt, a.k, a.m_rank, nq_wave, a.list_d + list_row, a.list_id + list_row, a.plane, tau_q0, tau_m_q0);
        __builtin_amdgcn_wave_barrier();
        if (lane < nq_wave) a.list_n[static_cast<size_t>(chunk) * a.n_q + q0 + lane] = W.ln[lane] | (W.par[lane] << 31);
    }
}

// ---- 3. merge of the chunk lists -------------------------------------------

__global__ __launch_bounds__(TK_MERGE_NT) void tk_merge(TkArgs a, const float* list_d, const uint32_t* list_id,
                                                         size_t plane, const uint32_t* list_n, uint32_t n_chunks,
                                                         uint32_t n_q, uint32_t k, float* out_d, int64_t* out_id)
{
    if (tk_small(a, tk_rows(a))) return;  // tk_select answers small sets
    constexpr int W = TK_MERGE_NT / 64;
    __shared__ float ad[W][2][TK_KMAX];
    __shared__ uint32_t ai[W][2][TK_KMAX];
    __shared__ float cd[W][TK_KMAX];
    __shared__ uint32_t ci[W][TK_KMAX];
    const uint32_t lane = __lane_id();
    const uint32_t w = threadIdx.x >> 6;
    const uint32_t q = blockIdx.x * W + w;
    if (q >= n_q) return;  // whole wave; no block barrier below
    uint32_t n = 0;
    int cur = 0;
    // The next chunk's list is loaded into registers (k <= 256: four entries a
    // lane) while the current one is merged.
    constexpr int PER = TK_KMAX / 64;
    float nd[PER];
    uint32_t ni[PER], nm = 0;
    auto fetch = [&](uint32_t c) {
        const size_t row = static_cast<size_t>(c) * n_q + q;
        const uint32_t ln = list_n[row];
        nm = ln & 0x7FFFFFFFu;
        const size_t base = (ln >> 31) * plane + row * k;
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const uint32_t i = lane + 64u * e;
            nd[e] = i < nm ? list_d[base + i] : 0.f;
            ni[e] = i < nm ? list_id[base + i] : 0u;
        }
    };
    if (n_chunks) fetch(0);
    for (uint32_t c = 0; c < n_chunks; ++c) {
        const uint32_t m = nm;
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const uint32_t i = lane + 64u * e;
            if (i < m) {
                cd[w][i] = nd[e];
                ci[w][i] = ni[e];
            }
        }
        if (c + 1 < n_chunks) fetch(c + 1);
        if (m == 0) continue;
        __builtin_amdgcn_wave_barrier();
        for (uint32_t i = lane; i < n; i += 64) {
            const float x = ad[w][cur][i];
            const uint32_t xi = ai[w][cur][i];
            const uint32_t r = i + tk_lower_bound(cd[w], ci[w], m, x, xi);
            if (r < k) {
                ad[w][cur ^ 1][r] = x;
                ai[w][cur ^ 1][r] = xi;
            }
        }
        for (uint32_t e = lane; e < m; e += 64) {
            const float y = cd[w][e];
            const uint32_t yi = ci[w][e];
            const uint32_t r = e + tk_lower_bound(ad[w][cur], ai[w][cur], n, y, yi);
            if (r < k) {
                ad[w][cur ^ 1][r] = y;
                ai[w][cur ^ 1][r] = yi;
            }
        }
        __builtin_amdgcn_wave_barrier();
        n = min(k, n + m);
        cur ^= 1;
    }
    for (uint32_t r = lane; r < k; r += 64) {
        out_d[static_cast<size_t>(q) * k + r] = r < n ? ad[w][cur][r] : __builtin_inff();
        out_id[static_cast<size_t>(q) * k + r] = r < n ? static_cast<int64_t>(ai[w][cur][r]) : int64_t(-1);
    }
}

// ---- 2b. small sets: every estimate ------------------------------------------
// The distance kernel's tiles and MFMA blocks without the selection: each
// (chunk, query block) workgroup writes the estimates of its rows for its
// queries -- (1 - TK_GATE_ERR)(|q|^2 + |x|^2) - 2 q.x, at most the fp32
// distance -- to pd[q][row], the scaled query norms to pq (chunk 0) and the
// scaled row norms to px (query block 0).
// Rows whose upper bounds set the first bound: a larger sample costs reads, a
// smaller one admits about k * rows / sample candidates, each a gathered row.
constexpr uint32_t TK_SEL_SAMPLE = 16384;
constexpr uint32_t TK_SEL_SAMPLE_PER_K = 1024;
// The upper bounds' range matters only over the rows a histogram reads: the
// selection's sample, which includes every seed row (at most 256 k of them).
__device__ __forceinline__ uint64_t tk_hist_rows(const TkArgs& a)
{
    return max(TK_SEL_SAMPLE, TK_SEL_SAMPLE_PER_K * a.k);
}

constexpr int TK_ES = TK_ROWS + 4;  // estimate staging: a query's 64 rows, 16-byte aligned

template <int DP>
struct TkPairsLds {
    float tile[2][TK_ROWS * (DP + 4)];
    float xg[2][TK_ROWS];
    uint32_t id[2][TK_ROWS];
    float est[TK_WAVES][TK_QW * TK_ES];  // a wave's 32 x 64 estimates
};

template <int DP, bool SEL>
__global__ __launch_bounds__(TK_NT) void tk_pairs(TkArgs a)
{
    // Every row of a small set, or the seed rows of a larger one.
    const uint64_t all_rows = tk_rows(a);
    const uint64_t n_rows = tk_small(a, all_rows) ? all_rows : tk_seed_rows(a, all_rows);
    if (n_rows == 0) return;
    __shared__ TkPairsLds<DP> L;
    const uint32_t lane = __lane_id();
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t h = lane >> 5;
    const uint32_t j = lane & 31u;
    // The workgroups of a query block take its tiles in turn: tile c, c + n_cw,
    // ... (the grid is n_cw x n_qb, balanced however many rows there are).
    const uint32_t n_qb = (a.n_q + TK_QB - 1) / TK_QB;
    const uint32_t n_cw = gridDim.x / n_qb;
    const uint32_t chunk = blockIdx.x / n_qb;
    const uint32_t qb = blockIdx.x % n_qb;
    const uint64_t n_all = (n_rows + TK_ROWS - 1) / TK_ROWS;
    const uint32_t n_tiles = chunk < n_all ? static_cast<uint32_t>((n_all - chunk + n_cw - 1) / n_cw) : 0u;
    auto tile_r0 = [&](uint32_t i) { return (static_cast<uint64_t>(chunk) + static_cast<uint64_t>(i) * n_cw) * TK_ROWS; };
    auto tile_r1 = [&](uint32_t i) { return std::min<uint64_t>(n_rows, tile_r0(i) + TK_ROWS); };
    const uint32_t q0 = qb * TK_QB + wave * TK_QW;
    const uint32_t uq0 = __builtin_amdgcn_readfirstlane(q0);  // the same, known to be wave-uniform
    const uint32_t nq_wave = q0 < a.n_q ? std::min<uint32_t>(TK_QW, a.n_q - q0) : 0u;
    const bool qok = j < nq_wave;
    float qreg[DP / 2];
    const float qpart = tk_load_query<DP>(a, qok, q0 + j, h, qreg);
    const float qg = (1.f - TK_GATE_ERR) * (qpart + __shfl_xor(qpart, 32, 64));
    if (chunk == 0 && h == 0 && qok) a.pq[q0 + j] = qg;
    float4 pre[DP / 32];
    uint32_t pid[DP / 32], nid[DP / 32];  // ids of the next tile, and (raw) of the one after it
    const uint64_t last = n_rows - 1;
    // A tile's loads are all issued before the previous tile's MFMA and
    // waited for after it: the rows of tile t + 1 (their ids known since
    // tile t - 1) and the ids of tile t + 2.  Every iteration prefetches (a tile
    // past the last has no valid rows and is never read), so no branch skips
    // a load and the one wait of an iteration comes after its MFMA.
    tk_ids_raw<DP, SEL>(a, tile_r0(1), last, nid);
    if (n_tiles > 0) {
        tk_load_rows<DP>(a, tile_r0(0), tile_r1(0), pre, pid);
        tk_store_rows<DP>(L, 0, pre, pid);
    }
#pragma unroll
    for (int p = 0; p < DP / 32; ++p) pid[p] = nid[p];
    tk_ids_valid<DP>(tile_r0(1), tile_r1(1), pid);
    __syncthreads();
    float ulo = __builtin_inff(), uhi = -__builtin_inff();  // range of the upper bounds of this lane's rows
    for (uint32_t t = 0; t < n_tiles; ++t) {
        const int b = static_cast<int>(t & 1u);
        tk_load_rows_nb<DP>(a, pid, pre);
        tk_ids_raw<DP, SEL>(a, tile_r0(t + 2), last, nid);
        if (nq_wave > 0) {
            f32x16 acc0 = {}, acc1 = {};
            const float* A0 = &L.tile[b][j * (DP + 4) + h * (DP / 2)];
            const float* A1 = A0 + 32 * (DP + 4);
#pragma unroll
            for (int s = 0; s < DP / 2; s += 4) {
                const float4 x0 = *reinterpret_cast<const float4*>(A0 + s);
                const float4 x1 = *reinterpret_cast<const float4*>(A1 + s);
                acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0.x, qreg[s + 0], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1.x, qreg[s + 0], acc1, 0, 0, 0);
                acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0.y, qreg[s + 1], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1.y, qreg[s + 1], acc1, 0, 0, 0);
                acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0.z, qreg[s + 2], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1.z, qreg[s + 2], acc1, 0, 0, 0);
                acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x0.w, qreg[s + 3], acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x1.w, qreg[s + 3], acc1, 0, 0, 0);
            }
            // Through LDS, so each store writes 64 consecutive rows of four
            // queries.  Accumulator registers 4m .. 4m + 3 of a block hold four
            // consecutive rows (tk_row), one 16-byte LDS access.
            float* E = L.est[wave];
            const int rows = static_cast<int>(tile_r1(t) - tile_r0(t));  // rows of this tile
            const bool track = tile_r0(t) < tk_hist_rows(a);  // uniform
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const int ra = tk_row(4 * m, static_cast<int>(h)), rb = tk_row(16 + 4 * m, static_cast<int>(h));
                const float4 ga = *reinterpret_cast<const float4*>(&L.xg[b][ra]);
                const float4 gb = *reinterpret_cast<const float4*>(&L.xg[b][rb]);
                const float4 ea = make_float4(qg + ga.x - 2.f * acc0[4 * m + 0], qg + ga.y - 2.f * acc0[4 * m + 1],
                                              qg + ga.z - 2.f * acc0[4 * m + 2], qg + ga.w - 2.f * acc0[4 * m + 3]);
                const float4 eb = make_float4(qg + gb.x - 2.f * acc1[4 * m + 0], qg + gb.y - 2.f * acc1[4 * m + 1],
                                              qg + gb.z - 2.f * acc1[4 * m + 2], qg + gb.w - 2.f * acc1[4 * m + 3]);
                *reinterpret_cast<float4*>(&E[j * TK_ES + ra]) = ea;
                *reinterpret_cast<float4*>(&E[j * TK_ES + rb]) = eb;
                if (track) {
                    const float e8[8] = {ea.x, ea.y, ea.z, ea.w, eb.x, eb.y, eb.z, eb.w};
                    const float g8[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
#pragma unroll
                    for (int c = 0; c < 8; ++c) {
                        const bool in = (c < 4 ? ra : rb - 4) + c < rows;  // a row of the tile
                        const float u = tk_upper(e8[c], qg, g8[c]);
                        ulo = fminf(ulo, in ? u : __builtin_inff());
                        uhi = fmaxf(uhi, in ? u : -__builtin_inff());
                    }
                }
            }
        }
        // Tile t + 1 into the other buffer, and tile t + 2's valid ids.
        tk_store_rows<DP>(L, b ^ 1, pre, pid);
#pragma unroll
        for (int p = 0; p < DP / 32; ++p) pid[p] = nid[p];
        tk_ids_valid<DP>(tile_r0(t + 2), tile_r1(t + 2), pid);
        // Every wave stores all 32 of its queries' rows and every lane its row
        // (the estimate rows are allocated for whole query blocks and whole
        // tiles; a query past n_q, or a row past the tile's last, receives a
        // value nothing reads), after the iteration's wait: nothing waits for
        // these stores before the next tile's MFMA has run.
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        {
            // lane l stores rows 4 (l % 16) .. + 3 of query 4 i + l / 16
            const float* E = L.est[wave];
            const uint32_t ql = lane >> 4, cl = 4u * (lane & 15u);
            float* dst = a.pd + static_cast<size_t>(uq0) * a.small_max + tile_r0(t);  // uniform
#pragma unroll
            for (uint32_t i = 0; i < TK_QW / 4; ++i) {
                const float4 v = *reinterpret_cast<const float4*>(&E[(4u * i + ql) * TK_ES + cl]);
                *reinterpret_cast<float4*>(dst + static_cast<size_t>(4u * i + ql) * a.small_max + cl) = v;
            }
            // the scaled norms, from every wave (the same values)
            a.px[tile_r0(t) + lane] = L.xg[b][lane];
        }
        __builtin_amdgcn_wave_barrier();
        __syncthreads();
    }
    ulo = fminf(ulo, __shfl_xor(ulo, 32, 64));
    uhi = fmaxf(uhi, __shfl_xor(uhi, 32, 64));
    if (h == 0 && qok && uhi >= ulo) {  // the lane pair saw at least one row
        atomicMin(a.qlo + q0 + j, tk_ordered(ulo));
        atomicMax(a.qhi + q0 + j, tk_ordered(uhi));
    }
}

// ---- 3b. small sets: one workgroup per query selects from every estimate ---
// Each row's estimate L is a lower bound of its fp32 distance and
// U = L + TK_SEED_ERR (qg + xg) an upper bound.  The k-th smallest U bounds the
// k-th smallest distance, so every row of the answer (ties included) has
// L <= that bound: those rows get their fp32 direct distance, are sorted by
// (distance, id) and the first k are written.
constexpr uint32_t TK_SMALL = 1u << 18;  // rows the small-set path takes at most
constexpr uint32_t TK_SMALL_BYTES = 1u << 30;  // and the estimates it may keep
constexpr int TK_SEL_NT = 1024;
constexpr uint32_t TK_SEL_BINS = TK_SEL_NT;  // one histogram bin per thread
constexpr uint32_t TK_SEL_CB = 8192;         // candidates per batch
constexpr uint32_t TK_SEL_RPT = 4;           // rows per thread per candidate chunk
// Process-wide limit of the small-set path (cr_topk_set_small_limit).
std::atomic<uint32_t> g_topk_small{TK_SMALL};

// A histogram of the upper bounds of rows [0, Sn) of the query's estimates
// over the range of all of them: the bins spread the values, so the counting
// atomics rarely collide.  The first bin at which the count reaches k holds the
// k-th smallest upper bound; the largest value in the bins up to it is the
// returned bound (at least k rows lie at or below it, so the k-th distance
// does).  Every thread of the workgroup calls it.
__device__ __forceinline__ float tk_hist_bound(const TkArgs& a, uint32_t q, const float* lrow, uint32_t Sn,
                                               uint32_t* hist, uint32_t* bmax, uint32_t* lds, uint32_t& s_bin,
                                               uint32_t& s_bound)
{
    const uint32_t t = threadIdx.x, lane = __lane_id();
    const float qg = a.pq[q];
    const float vlo = tk_unordered(a.qlo[q]), vhi = tk_unordered(a.qhi[q]);
    const float scale = vhi > vlo ? static_cast<float>(TK_SEL_BINS) / (vhi - vlo) : 0.f;
    hist[t] = 0;
    bmax[t] = 0;
    if (t == 0) s_bound = 0;
    __syncthreads();
    // Eight rows a thread per step, the next step's loads issued before this
    // step's are binned (clamped to the last row, tested against Sn only where
    // used, so nothing waits for them early).
    const uint32_t last = Sn - 1;  // Sn > k >= 1
    float l8[8], x8[8];
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
        const uint32_t r = min(t + i * TK_SEL_NT, last);
        l8[i] = lrow[r];
        x8[i] = a.px[r];
    }
    for (uint32_t r0 = t; r0 < Sn; r0 += 8 * TK_SEL_NT) {
        float nl8[8], nx8[8];
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i) {
            const uint32_t r = min(r0 + (8 + i) * TK_SEL_NT, last);
            nl8[i] = lrow[r];
            nx8[i] = a.px[r];
        }
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i) {
            if (r0 + i * TK_SEL_NT >= Sn) break;
            const float u = tk_upper(l8[i], qg, x8[i]);
            const float f = (u - vlo) * scale;
            const uint32_t bin = f >= static_cast<float>(TK_SEL_BINS - 1) ? TK_SEL_BINS - 1
                                                                          : static_cast<uint32_t>(fmaxf(f, 0.f));
            atomicAdd(&hist[bin], 1u);
            atomicMax(&bmax[bin], tk_ordered(u));
        }
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i) l8[i] = nl8[i], x8[i] = nx8[i];
    }
    __syncthreads();
    uint32_t total;
    const uint32_t h = hist[t];
    const uint32_t excl = block_excl_scan<TK_SEL_NT>(h, lds, total);
    if (excl < a.k && excl + h >= a.k) s_bin = t;
    __syncthreads();
    uint32_t m = t <= s_bin ? bmax[t] : 0u;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = max(m, static_cast<uint32_t>(__shfl_xor(m, o, 64)));
    if (lane == 0 && m) atomicMax(&s_bound, m);
    __syncthreads();
    return tk_unordered(s_bound);
}

// One workgroup per query, right after tk_pairs, on both paths.  A small set
// is answered here (below).  A larger one gets query q's bound from the upper
// bounds of its seed rows (more than k of them), into tau for the list path:
// at least k rows have an fp32 distance at or below it, so the k-th best does
// (tau holds the bits of non-negative distances).
__global__ __launch_bounds__(TK_SEL_NT) __attribute__((amdgpu_waves_per_eu(8))) void tk_select(TkArgs a, float* out_d, int64_t* out_id)
{
    __shared__ float bd[2][TK_KMAX];  // the running best, ascending (two planes)
    __shared__ uint32_t bi[2][TK_KMAX];
    __shared__ float cd[TK_SEL_CB];  // a batch of candidates
    __shared__ uint32_t ci[TK_SEL_CB];
    __shared__ uint32_t hist[TK_SEL_BINS], bmax[TK_SEL_BINS];
    __shared__ float qv[128];
    __shared__ uint32_t lds[TK_SEL_NT / 64];
    __shared__ uint32_t s_bin, s_bound, s_nbatch;
    const uint64_t n_rows = tk_rows(a);
    // More rows than the small-set limit with no list path launched: only a
    // filter whose recorded cardinality understates its set does that, and
    // every row is then a candidate (exact, slower; no estimate is read).
    const bool all_rows = a.list_off && !tk_small(a, n_rows);
    if (!tk_small(a, n_rows) && !all_rows) {  // the list path answers; its seed bound
        const uint32_t Sd = tk_seed_rows(a, n_rows);
        if (Sd <= a.k) return;
        const uint32_t qs = blockIdx.x;
        const float sb = tk_hist_bound(a, qs, a.pd + static_cast<size_t>(qs) * a.small_max, Sd, hist, bmax, lds,
                                       s_bin, s_bound);
        if (threadIdx.x == 0) atomicMin(a.tau + qs, __float_as_uint(fmaxf(sb, 0.f)));
        return;
    }
    const uint32_t S = static_cast<uint32_t>(n_rows);
    const uint32_t q = blockIdx.x;
    const uint32_t t = threadIdx.x;
    const float* lrow = a.pd + static_cast<size_t>(q) * a.small_max;
    for (uint32_t c = t; c < 128; c += TK_SEL_NT) qv[c] = c < a.dim ? a.queries[static_cast<size_t>(q) * a.dim + c] : 0.f;
    float bound = __builtin_inff();
    if (S > a.k && !all_rows) {
        // The first bound from the upper bounds of the first rows (a sample
        // only loosens it).
        const uint32_t Sn = min(S, max(TK_SEL_SAMPLE, TK_SEL_SAMPLE_PER_K * a.k));
        bound = tk_hist_bound(a, q, lrow, Sn, hist, bmax, lds, s_bin, s_bound);
    }
    // Candidates (rows whose estimate, a lower bound, is at or below the bound)
    // in batches: fp32 direct distances, a sort by (distance, id), and a merge
    // into the running best k.
    uint32_t nb = 0, cur = 0, nbatch = 0;
    auto flush = [&]() {
        __syncthreads();  // the batch's rows are in ci
        for (uint32_t c0 = 0; c0 < nbatch; c0 += TK_SEL_NT / 8) {  // eight threads per candidate
            const uint32_t c = c0 + t / 8, part = t % 8;
            float e2 = 0.f;
            uint32_t id = 0;
            if (c < nbatch) {
                const uint32_t r = ci[c];
                id = a.sel ? a.sel[r] : r;
                // the part's 16 dimensions, all loaded before any is used (zeros
                // past dim, where qv is zero too, add nothing)
                const float* x = a.base + static_cast<size_t>(id) * a.dim + part * 16;
#pragma unroll
                for (uint32_t hh = 0; hh < 16; hh += 8) {  // two halves of 8
                    float xv[8];
                    if (a.vec) {  // dim % 4 == 0, 16-byte aligned rows
#pragma unroll
                        for (uint32_t q4 = 0; q4 < 8; q4 += 4) {
                            const float4 v = part * 16 + hh + q4 < a.dim
                                                 ? *reinterpret_cast<const float4*>(x + hh + q4)
                                                 : make_float4(0.f, 0.f, 0.f, 0.f);
                            xv[q4] = v.x, xv[q4 + 1] = v.y, xv[q4 + 2] = v.z, xv[q4 + 3] = v.w;
                        }
                    } else {
#pragma unroll
                        for (uint32_t s2 = 0; s2 < 8; ++s2) xv[s2] = part * 16 + hh + s2 < a.dim ? x[hh + s2] : 0.f;
                    }
#pragma unroll
                    for (uint32_t s2 = 0; s2 < 8; ++s2) {
                        const float e = qv[part * 16 + hh + s2] - xv[s2];
                        e2 = fmaf(e, e, e2);
                    }
                }
            }
            e2 += __shfl_xor(e2, 1, 64);
            e2 += __shfl_xor(e2, 2, 64);
            e2 += __shfl_xor(e2, 4, 64);
            __syncthreads();  // every thread of the pass has read ci[c]
            if (c < nbatch && part == 0) {
                cd[c] = e2;
                ci[c] = id;
            }
        }
        uint32_t P = 2;
        while (P < nbatch) P <<= 1;
        __syncthreads();
        for (uint32_t i = nbatch + t; i < P; i += TK_SEL_NT) {
            cd[i] = __builtin_inff();
            ci[i] = TK_NOID;
        }
        __syncthreads();
        for (uint32_t size = 2; size <= P; size <<= 1) {
            for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
                for (uint32_t i = t; i < P / 2; i += TK_SEL_NT) {
                    const uint32_t lo = 2 * i - (i & (stride - 1));
                    const uint32_t hi = lo + stride;
                    const bool up = (lo & size) == 0;
                    const float dl = cd[lo], dh = cd[hi];
                    const uint32_t il = ci[lo], ih = ci[hi];
                    if (tk_less(dh, ih, dl, il) == up) {
                        cd[lo] = dh;
                        cd[hi] = dl;
                        ci[lo] = ih;
                        ci[hi] = il;
                    }
                }
                __syncthreads();
            }
        }
        // Merge: an entry's rank is its index plus the number of entries of
        // the other list before it (all (distance, id) pairs are distinct).
        const uint32_t nbt = min(nbatch, a.k);
        if (t < nb) {
            const uint32_t r = t + tk_lower_bound(cd, ci, nbt, bd[cur][t], bi[cur][t]);
            if (r < a.k) {
                bd[cur ^ 1][r] = bd[cur][t];
                bi[cur ^ 1][r] = bi[cur][t];
            }
        } else if (t - nb < nbt) {
            const uint32_t e = t - nb;
            const uint32_t r = e + tk_lower_bound(bd[cur], bi[cur], nb, cd[e], ci[e]);
            if (r < a.k) {
                bd[cur ^ 1][r] = cd[e];
                bi[cur ^ 1][r] = ci[e];
            }
        }
        nb = min(a.k, nb + nbt);
        cur ^= 1;
        nbatch = 0;
        if (t == 0) s_nbatch = 0;
        __syncthreads();
        if (nb == a.k) bound = fminf(bound, bd[cur][a.k - 1]);  // the k-th best so far bounds the answer
    };
    // Candidates are few: a thread that finds one takes a batch slot with an
    // LDS atomic.  Chunks of TK_SEL_RPT consecutive rows per thread (one
    // 16-byte load), the loads of the next two chunks in flight while one is
    // tested (clamped to the last whole vector of the row, which the estimate
    // row holds, and tested against S only where used, so nothing waits for
    // them early); a batch that could overflow in the next chunk is flushed
    // first.
    static_assert(TK_SEL_RPT == 4, "one float4 a thread per chunk");
    constexpr uint32_t CH = TK_SEL_RPT * TK_SEL_NT;
    if (t == 0) s_nbatch = 0;
    if (all_rows) {
        for (uint32_t r0 = 0; r0 < S; r0 += CH) {
            __syncthreads();  // the previous chunk's slots are taken
            nbatch = s_nbatch;
            __syncthreads();
            if (nbatch > TK_SEL_CB - CH) flush();
#pragma unroll
            for (uint32_t i = 0; i < TK_SEL_RPT; ++i) {
                const uint32_t r = r0 + i * TK_SEL_NT + t;
                if (r < S) ci[atomicAdd(&s_nbatch, 1u)] = r;
            }
        }
    }
    const uint32_t last4 = S > 0 && !all_rows ? (S - 1) & ~3u : 0;
    auto ld4 = [&](uint32_t r) { return *reinterpret_cast<const float4*>(lrow + min(r, last4)); };
    float4 l4 = ld4(4 * t), n4 = ld4(CH + 4 * t);
    for (uint32_t r0 = 0; r0 < (all_rows ? 0u : S); r0 += CH) {
        const float4 m4 = ld4(r0 + 2 * CH + 4 * t);
        __syncthreads();  // the previous chunk's slots are taken
        nbatch = s_nbatch;
        __syncthreads();  // every thread has read the count before the next slots are taken
        if (nbatch > TK_SEL_CB - CH) flush();
        const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            const uint32_t r = r0 + 4 * t + i;
            if (r < S && lv[i] <= bound) ci[atomicAdd(&s_nbatch, 1u)] = r;
        }
        l4 = n4;
        n4 = m4;
    }
    __syncthreads();
    nbatch = s_nbatch;
    if (nbatch) flush();
    for (uint32_t r = t; r < a.k; r += TK_SEL_NT) {
        const bool ok = r < nb;
        out_d[static_cast<size_t>(q) * a.k + r] = ok ? bd[cur][r] : __builtin_inff();
        out_id[static_cast<size_t>(q) * a.k + r] = ok ? static_cast<int64_t>(bi[cur][r]) : int64_t(-1);
    }
}

// The call's state (tk_init_from), when no enumeration kernel sets it.
__global__ __launch_bounds__(256) void tk_init(TkArgs a)
{
    tk_init_from(a, static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x, static_cast<uint64_t>(gridDim.x) * 256u);
}

template <int DP>
int launch_dist(const TkArgs& a, uint32_t grid, uint32_t pairs_grid, float* out_d, int64_t* out_ids, hipStream_t s)
{
    if (a.small_max) {  // estimates of a small set (and its answer), or the seed rows of a larger one and their bound
        {
            CR_TIMED("tk_pairs", s);
            if (a.sel)
                tk_pairs<DP, true><<<pairs_grid, TK_NT, 0, s>>>(a);
            else
                tk_pairs<DP, false><<<pairs_grid, TK_NT, 0, s>>>(a);
        }
        CR_LAUNCH_CHECK();
        {
            CR_TIMED("tk_select", s);
            tk_select<<<a.n_q, TK_SEL_NT, 0, s>>>(a, out_d, out_ids);
        }
        CR_LAUNCH_CHECK();
    }
    if (!a.list_off) {
        CR_TIMED("tk_dist", s);
        if (a.sel)
            tk_dist<DP, true><<<grid, TK_NT, 0, s>>>(a);
        else
            tk_dist<DP, false><<<grid, TK_NT, 0, s>>>(a);
    }
    CR_LAUNCH_CHECK();
    return CR_OK;
}

}  // namespace
}  // namespace crimpl

using namespace crimpl;

extern "C" int cr_topk_filtered(const float* d_base, uint64_t n_base, const float* d_queries, uint32_t n_q,
                                uint32_t dim, const cr_gpu_roaring* filter, uint32_t k, float* d_out_dist,
                                int64_t* d_out_ids, cr_stream_t stream)
{
    if (n_q == 0 || k == 0) return CR_OK;
    if (!d_queries || !d_out_dist || !d_out_ids || (n_base && !d_base) || dim == 0) {
        set_error("cr_topk_filtered: invalid argument");
        return CR_ERR_INVALID;
    }
    if (dim > 128 || k > TK_KMAX || n_base > 0xFFFFFFFFull) {
        set_error("cr_topk_filtered: supported up to dim 128, k %u and 2^32-1 base vectors (dim %u, k %u)", TK_KMAX,
                  dim, k);
        return CR_ERR_UNSUPPORTED;
    }
    hipStream_t s = as_stream(stream);
    const uint32_t n_qb = (n_q + TK_QB - 1) / TK_QB;
    // Enough (chunk, query block) workgroups to cover every CU once.
    const uint32_t cus = num_cus();
    uint32_t n_chunks = std::max<uint32_t>(8, (cus + n_qb - 1) / n_qb);
    n_chunks = (n_chunks + 7) / 8 * 8;
    const uint64_t nb = (n_base + TK_ENUM_IDS - 1) / TK_ENUM_IDS;

    Carver cv;
    const size_t o_counts = cv.add(filter ? nb * 4 : 0);
    const size_t o_nsel = cv.add(4);
    const size_t o_sel = cv.add(filter ? n_base * 4 : 0);
    const size_t lists = static_cast<size_t>(n_chunks) * n_q * k;
    const size_t o_ld = cv.add(2 * lists * 4);
    const size_t o_li = cv.add(2 * lists * 4);
    const size_t o_ln = cv.add(static_cast<size_t>(n_chunks) * n_q * 4);
    const size_t o_tau = cv.add(static_cast<size_t>(n_q) * 4);
    const size_t o_taum = cv.add(static_cast<size_t>(n_chunks) * n_q * 4);
    // The small-set path keeps every estimate, small_max floats for each query
    // of every whole query block, within TK_SMALL_BYTES.
    const uint64_t q_rows = static_cast<uint64_t>(n_qb) * TK_QB;
    const uint32_t small_max = static_cast<uint32_t>(std::min<uint64_t>(
        g_topk_small.load(), TK_SMALL_BYTES / (4ull * q_rows) / TK_ROWS * TK_ROWS));
    const size_t o_pd = cv.add(q_rows * small_max * 4);
    const size_t o_pq = cv.add(small_max ? static_cast<size_t>(n_q) * 4 : 0);
    const size_t o_px = cv.add(static_cast<size_t>(small_max) * 4);
    const size_t o_qlo = cv.add(small_max ? static_cast<size_t>(n_q) * 4 : 0);
    const size_t o_qhi = cv.add(small_max ? static_cast<size_t>(n_q) * 4 : 0);
    Scratch sc;
    CR_RET(sc.alloc(cv.total, s));

    TkArgs a{};
    a.base = d_base;
    a.queries = d_queries;
    a.n_base = n_base;
    a.n_q = n_q;
    a.dim = dim;
    a.k = k;
    a.n_chunks = n_chunks;
    a.vec = (dim % 4 == 0) && (reinterpret_cast<uintptr_t>(d_base) % 16 == 0);
    a.qvec = (dim % 4 == 0) && (reinterpret_cast<uintptr_t>(d_queries) % 16 == 0);
    a.list_d = sc.at<float>(o_ld);
    a.list_id = sc.at<uint32_t>(o_li);
    a.list_n = sc.at<uint32_t>(o_ln);
    a.plane = lists;
    a.tau = sc.at<uint32_t>(o_tau);
    a.tau_m = sc.at<uint32_t>(o_taum);
    a.m_rank = std::max<uint32_t>(1, (2 * k + n_chunks - 1) / n_chunks);
    a.small_max = small_max;
    a.pd = small_max ? sc.at<float>(o_pd) : nullptr;
    a.pq = small_max ? sc.at<float>(o_pq) : nullptr;
    a.px = small_max ? sc.at<float>(o_px) : nullptr;
    a.qlo = small_max ? sc.at<uint32_t>(o_qlo) : nullptr;
    a.qhi = small_max ? sc.at<uint32_t>(o_qhi) : nullptr;
    // The list path is not launched when the passing count is known to fit the
    // small-set path: no filter and a small base, or a filter's recorded
    // cardinality (the library's uploads and fused multi_and record it, and the
    // reference's conversions rely on it too, src/to_csr.cu:212-216), plus one
    // per container for a multi_and's full containers stored as 65535.
    if (small_max) {
        const uint64_t bound = !filter ? n_base
                                       : (filter->total_cardinality > 0
                                              ? std::min<uint64_t>(n_base, filter->total_cardinality + filter->n_containers)
                                              : UINT64_MAX);
        a.list_off = bound <= small_max ? 1u : 0u;
    }
    if (!filter || nb == 0) {
        tk_init<<<static_cast<unsigned>((static_cast<uint64_t>(n_chunks) * n_q + 255) / 256), 256, 0, s>>>(a);
        CR_LAUNCH_CHECK();
    }
    if (filter) {
        cr_gpu_roaring_view cv_view;
        CR_RET(cr_make_view(filter, &cv_view));
        GpuRoaringView v;
        static_assert(sizeof(v) == sizeof(cv_view), "view layout");
        std::memcpy(&v, &cv_view, sizeof(v));
        a.sel = sc.at<uint32_t>(o_sel);
        a.n_sel = sc.at<uint32_t>(o_nsel);
        if (nb == 0) {
            CR_RET(fill_u32(sc.at<uint32_t>(o_nsel), 0u, 1, s));
        } else {
            CR_TIMED("tk_enum", s);
            tk_enum_count<<<static_cast<unsigned>(nb), TK_ENUM_NT, 0, s>>>(v, n_base, sc.at<uint32_t>(o_counts), a);
            tk_enum_write<<<static_cast<unsigned>(nb), TK_ENUM_NT, 0, s>>>(v, n_base, sc.at<uint32_t>(o_counts),
                                                                           sc.at<uint32_t>(o_sel), sc.at<uint32_t>(o_nsel));
        }
        CR_LAUNCH_CHECK();
    }
    const uint32_t grid = n_chunks * n_qb;
    // tk_pairs: one workgroup a CU (two waves a SIMD fill it), each query
    // block's tiles dealt out among its workgroups
    const uint32_t pairs_grid = std::max<uint32_t>(1, (cus + n_qb - 1) / n_qb) * n_qb;
    if (dim <= 32) {
        CR_RET(launch_dist<32>(a, grid, pairs_grid, d_out_dist, d_out_ids, s));
    } else if (dim <= 64) {
        CR_RET(launch_dist<64>(a, grid, pairs_grid, d_out_dist, d_out_ids, s));
    } else {
        CR_RET(launch_dist<128>(a, grid, pairs_grid, d_out_dist, d_out_ids, s));
    }
    if (!a.list_off) {
        CR_TIMED("tk_merge", s);
        tk_merge<<<(n_q + 3) / 4, TK_MERGE_NT, 0, s>>>(a, a.list_d, a.list_id, a.plane, a.list_n, n_chunks, n_q, k,
                                                        d_out_dist, d_out_ids);
    }
    CR_LAUNCH_CHECK();
    return CR_OK;
}

extern "C" uint32_t cr_topk_set_small_limit(uint32_t rows)
{
    const uint32_t prev = g_topk_small.load();
    g_topk_small.store(std::min<uint32_t>(rows, TK_SMALL));
    return prev;
}

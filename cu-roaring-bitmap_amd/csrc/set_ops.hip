// set_operation and multi_and on gfx950.
//
// Semantics follow src/set_ops.cu (reference): DeMorgan rewrite (:533-565),
// key matching (:76-122), pair classification and output container types
// (:626-692), pool slot order (:695-701, :864-886, :1005-1010), zero-card drop
// rules (:1038-1159), fused all-bitmap multi_and (:1489-1710) and routing
// (:1715-1745).  The structure is new: container matching runs on the device
// over the 65536-key space (one thread per key), every pair type runs in one
// grid-stride kernel (one workgroup per output container), and the output
// metadata is compacted on the device, so a call costs one host sync (its
// output is sized from the inputs' container counts) instead of the
// reference's per-class round trips.
#include <algorithm>

#include "image.hpp"
#include "internal.hpp"

namespace crimpl {

enum : uint8_t { CAT_NONE = 0, CAT_BB, CAT_BA, CAT_AA, CAT_MIXED, CAT_COPY_BMP, CAT_COPY_ARR, CAT_COPY_RUN };

// Per-key classification record (plan pass 1).
struct KeyRec {
    uint8_t cat;
    uint8_t pad[3];
    int32_t ai, bi;
    uint32_t size;        // array elements or run pairs reserved in the output pool
    uint32_t aoff, boff;  // byte offsets of the source containers
    uint32_t ma, mb;      // (type << 16) | stored card of the source containers, 0 when absent
};

// One output container candidate, in key order (plan pass 2).
struct Item {
    uint16_t key;
    uint8_t cat;
    uint8_t pad;
    int32_t ai, bi;
    uint32_t slot;        // bitmap slot, or u16 element offset into the array / run pool
    uint32_t aoff, boff;  // byte offsets of the source containers (0 when absent)
    uint32_t ma, mb;      // (type << 16) | stored card of the source containers (0 when absent)
};
static_assert(sizeof(Item) == 32, "the plans write an item as two 16-byte words");

// An item as the execution reads it (one scalar load): in execution order, with
// its position in key order, where its card goes.
struct ExecItem {
    uint16_t pos;    // position in key order (< 65536: one item a key)
    uint8_t cat;
    uint8_t from_a;  // a one-sided item's side
    uint32_t slot;
    uint32_t aoff, boff;
    uint32_t ma, mb;
    // A side that is a run container of one run: that run's word (start |
    // length - 1 << 16), so the execution needs no load of its payload; else 0.
    uint32_t run0_a, run0_b;
};
static_assert(sizeof(ExecItem) == 32, "one 32-byte scalar load");

// Counters accumulated per 1024-key group and totalled over all groups.  The
// last three check the key indexes when the classification reads them: the keys
// each side's index names (entries below n_containers) and the named keys whose
// container holds another key.
enum { C_ITEM, C_BB, C_MX, C_CB, C_BAE, C_AAE, C_CAE, C_CRP, C_BA, C_AA, C_CA, C_CR, C_KA, C_KB, C_KBAD, C_N };

struct Totals {
    uint32_t c[C_N];
    uint32_t n_out;     // containers kept after the zero-card drop
    uint32_t overflow;  // the plan needs more output than the caller's capacity
    uint32_t pad[2];
};

// What the host reads after the call's one synchronisation (a pinned slot).
struct SetOpHost {
    uint32_t c[C_N];
    uint32_t n_out;
    uint32_t overflow;
};

// Output capacity the host allocated before planning: work items (metadata
// entries), bitmap slots, array elements, run u16s.  0xFFFFFFFF = unbounded.
// `items` also bounds the plan's own item scratch, so it is never unbounded.
struct Caps {
    uint32_t items, bmp, arr, run_u16;
    uint32_t bb_only;  // the host launches the bitmap-only kernel: every item must be BB or COPY_BMP
    // With check_kidx the classification read both key indexes: the plan is
    // only valid if they name exactly na and nb keys, each the key its
    // container holds (the reference matches on `keys`, src/set_ops.cu:76-122).
    uint32_t check_kidx, na, nb;
    // Items that write array or run values, at most: the execution launches
    // waves for this many (and for `bmp` bitmap-writing ones).
    uint32_t small;
};

// The classification reads the key indexes instead of searching the keys.
__host__ __device__ inline bool use_kidx(const uint16_t* kidx_a, uint32_t na, const uint16_t* kidx_b, uint32_t nb)
{
    return kidx_a && kidx_b && na < 0xFFFFu && nb < 0xFFFFu;
}

struct Side {  // the parts of a GpuRoaring the kernels read
    const uint16_t* keys;
    const uint8_t* types;
    const uint32_t* offsets;
    const uint16_t* cards;
    const uint64_t* bmp;
    const uint16_t* arr;
    const uint16_t* run;
    uint32_t n;
    const uint16_t* kidx;  // key -> container index (0xFFFF: absent) for keys <= max_key, or null
    uint32_t kidx_n;       // max_key + 1 with kidx
};

static Side side_of(const cr_gpu_roaring* r)
{
    return Side{r->keys, r->types, r->offsets, r->cardinalities, r->bitmap_data, r->array_data, r->run_data,
                r->n_containers, r->key_index, r->key_index ? r->max_key + 1u : 0u};
}

constexpr int PLAN_NT = 1024;
constexpr int PLAN_GROUPS = 65536 / PLAN_NT;

// ---- plan pass 1: classify every key -------------------------------------
__global__ __launch_bounds__(PLAN_NT) void so_plan_classify(Side A, Side B, uint32_t op, KeyRec* recs,
                                                            uint32_t* group_counts)
{
    __shared__ int32_t ia[PLAN_NT], ib[PLAN_NT];
    __shared__ uint32_t range[4];
    __shared__ uint32_t red[C_N * (PLAN_NT / 64)];
    const uint32_t base = blockIdx.x * PLAN_NT;
    const uint32_t t = threadIdx.x;
    int32_t ai, bi;
    uint32_t cnt[C_N] = {};
    if (use_kidx(A.kidx, A.n, B.kidx, B.n)) {
        // Both sides index their keys (and 0xFFFF cannot be a real index):
        // one coalesced load a side, no search of the keys.  Each named key is
        // checked against its container's key, and the named keys are counted;
        // the plan flags an index that does not describe `keys` exactly.
        const uint32_t key = base + t;
        auto look = [&](const Side& S) -> int32_t {
            const uint32_t x = key < S.kidx_n ? S.kidx[key] : 0xFFFFu;
            return x < S.n ? static_cast<int32_t>(x) : -1;
        };
        ai = look(A);
        bi = look(B);
        cnt[C_KA] = ai >= 0 ? 1u : 0u;
        cnt[C_KB] = bi >= 0 ? 1u : 0u;
        cnt[C_KBAD] = (ai >= 0 && A.keys[ai] != key) || (bi >= 0 && B.keys[bi] != key) ? 1u : 0u;
    } else {
        const uint32_t wv = t >> 6;  // waves 0-3: the key range of this group in A and in B
        if (wv < 4) {
            const uint32_t r = wave_lower_bound_u16(wv < 2 ? A.keys : B.keys, wv < 2 ? A.n : B.n,
                                                    base + ((wv & 1u) ? PLAN_NT : 0u));
            if ((t & 63u) == 0) range[wv] = r;
        }
        ia[t] = -1;
        ib[t] = -1;
        __syncthreads();
        for (uint32_t j = range[0] + t; j < range[1]; j += PLAN_NT) {
            const uint32_t k = A.keys[j] - base;  // in range for sorted keys; guarded for malformed input
            if (k < PLAN_NT) ia[k] = static_cast<int32_t>(j);
        }
        for (uint32_t j = range[2] + t; j < range[3]; j += PLAN_NT) {
            const uint32_t k = B.keys[j] - base;
            if (k < PLAN_NT) ib[k] = static_cast<int32_t>(j);
        }
        __syncthreads();
        ai = ia[t];
        bi = ib[t];
    }
    KeyRec rec{};
    rec.ai = ai;
    rec.bi = bi;
    rec.aoff = ai >= 0 ? A.offsets[ai] : 0u;
    rec.boff = bi >= 0 ? B.offsets[bi] : 0u;
    const uint32_t ta = ai >= 0 ? A.types[ai] : 0u, tb = bi >= 0 ? B.types[bi] : 0u;
    const uint32_t ca = ai >= 0 ? A.cards[ai] : 0u, cb = bi >= 0 ? B.cards[bi] : 0u;
    rec.ma = ai >= 0 ? (ta << 16) | ca : 0u;
    rec.mb = bi >= 0 ? (tb << 16) | cb : 0u;
    const bool keep_a_only = op != CR_AND;                 // OR, XOR, ANDNOT copy A-only keys
    const bool keep_b_only = op == CR_OR || op == CR_XOR;  // OR, XOR copy B-only keys
    if (ai >= 0 && bi >= 0) {
        if (ta == CR_BITMAP && tb == CR_BITMAP) {
            rec.cat = CAT_BB;
            cnt[C_BB] = 1;
        } else if (op == CR_AND && ((ta == CR_BITMAP && tb == CR_ARRAY) || (ta == CR_ARRAY && tb == CR_BITMAP))) {
            rec.cat = CAT_BA;
            rec.size = ta == CR_ARRAY ? ca : cb;
            cnt[C_BAE] = rec.size;
            cnt[C_BA] = 1;
        } else if (op == CR_AND && ta == CR_ARRAY && tb == CR_ARRAY) {
            rec.cat = CAT_AA;
            rec.size = min(ca, cb);
            cnt[C_AAE] = rec.size;
            cnt[C_AA] = 1;
        } else {
            rec.cat = CAT_MIXED;
            cnt[C_MX] = 1;
        }
    } else if ((ai >= 0 && keep_a_only) || (bi >= 0 && keep_b_only)) {
        const bool from_a = ai >= 0;
        const uint32_t ty = from_a ? ta : tb;
        const uint32_t c = from_a ? ca : cb;
        if (ty == CR_BITMAP) {
            rec.cat = CAT_COPY_BMP;
            cnt[C_CB] = 1;
        } else if (ty == CR_ARRAY) {
            rec.cat = CAT_COPY_ARR;
            rec.size = c;
            cnt[C_CAE] = c;
            cnt[C_CA] = 1;
        } else {
            rec.cat = CAT_COPY_RUN;
            rec.size = c;
            cnt[C_CRP] = c;
            cnt[C_CR] = 1;
        }
    }
    if (rec.cat != CAT_NONE) cnt[C_ITEM] = 1;
    recs[base + t] = rec;
    // The group's counters: wave sums (DPP), then one thread per counter over
    // the waves -- a single barrier.
    constexpr uint32_t NW = PLAN_NT / 64;
#pragma unroll
    for (int k = 0; k < C_N; ++k) {
        const uint32_t ws = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(wave_incl_scan(cnt[k])), 63));
        if (__lane_id() == 0) red[k * NW + (t >> 6)] = ws;
    }
    __syncthreads();
    if (t < C_N) {
        uint32_t sum = 0;
#pragma unroll
        for (uint32_t i = 0; i < NW; ++i) sum += red[t * NW + i];
        group_counts[blockIdx.x * C_N + t] = sum;
    }
}

// ---- plan pass 2: slot assignment in key order -----------------------------
__global__ __launch_bounds__(PLAN_NT) void so_plan_assign(const KeyRec* recs, const uint32_t* group_counts,
                                                          Item* items, ExecItem* xitems, Totals* totals, Caps caps,
                                                          const uint16_t* run_a, const uint16_t* run_b)
{
    __shared__ uint32_t gbase[C_N], gtot[C_N];
    __shared__ uint32_t scan_lds[2 * 8 * (PLAN_NT / 64) + 8];
    const uint32_t t = threadIdx.x;
    static_assert(PLAN_GROUPS == 64 && C_N <= PLAN_NT / 64, "one wave per counter, one lane per group");
    if ((t >> 6) < C_N) {  // wave k: counter k over the 64 groups, before this one and in total
        const uint32_t k = t >> 6, g = __lane_id();
        const uint32_t v = group_counts[g * C_N + k];
        const uint32_t sb = static_cast<uint32_t>(
            __builtin_amdgcn_readlane(static_cast<int>(wave_incl_scan(g < blockIdx.x ? v : 0u)), 63));
        const uint32_t st = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(wave_incl_scan(v)), 63));
        if (g == 0) gbase[k] = sb, gtot[k] = st;
    }
    __syncthreads();
    if (blockIdx.x == 0 && t < C_N) totals->c[t] = gtot[t];
    if (blockIdx.x == 0 && t == C_N) totals->n_out = 0;
    if (blockIdx.x == 0 && t == C_N + 1)
        totals->overflow = gtot[C_ITEM] > caps.items || gtot[C_BB] + gtot[C_MX] + gtot[C_CB] > caps.bmp ||
                           gtot[C_BAE] + gtot[C_AAE] + gtot[C_CAE] > caps.arr || 2u * gtot[C_CRP] > caps.run_u16 ||
                           (caps.bb_only && gtot[C_BB] + gtot[C_CB] != gtot[C_ITEM]) ||
                           gtot[C_ITEM] - (gtot[C_BB] + gtot[C_MX] + gtot[C_CB]) > caps.small ||
                           (caps.check_kidx && (gtot[C_KA] != caps.na || gtot[C_KB] != caps.nb || gtot[C_KBAD] != 0));

    const uint32_t key = blockIdx.x * PLAN_NT + t;
    const KeyRec rec = recs[key];
    const uint8_t cat = rec.cat;
    // Per-thread contributions to the counters that define positions, scanned
    // over the group together.
    uint32_t pv[8] = {cat != CAT_NONE ? 1u : 0u,
                      cat == CAT_BB ? 1u : 0u,
                      cat == CAT_MIXED ? 1u : 0u,
                      cat == CAT_COPY_BMP ? 1u : 0u,
                      cat == CAT_BA ? rec.size : 0u,
                      cat == CAT_AA ? rec.size : 0u,
                      cat == CAT_COPY_ARR ? rec.size : 0u,
                      cat == CAT_COPY_RUN ? rec.size : 0u};
    uint32_t ptot[8];
    block_excl_scan_multi<PLAN_NT, 8>(pv, scan_lds, ptot);
    const uint32_t item_pos = gbase[C_ITEM] + pv[0];
    const uint32_t p_bb = pv[1], p_mx = pv[2], p_cb = pv[3], p_ba = pv[4], p_aa = pv[5], p_ca = pv[6], p_cr = pv[7];
    if (cat == CAT_NONE) return;
    uint32_t slot = 0;
    switch (cat) {
    case CAT_BB: slot = gbase[C_BB] + p_bb; break;
    case CAT_MIXED: slot = gtot[C_BB] + gbase[C_MX] + p_mx; break;
    case CAT_COPY_BMP: slot = gtot[C_BB] + gtot[C_MX] + gbase[C_CB] + p_cb; break;
    case CAT_BA: slot = gbase[C_BAE] + p_ba; break;
    case CAT_AA: slot = gtot[C_BAE] + gbase[C_AAE] + p_aa; break;
    case CAT_COPY_ARR: slot = gtot[C_BAE] + gtot[C_AAE] + gbase[C_CAE] + p_ca; break;
    default: slot = 2u * (gbase[C_CRP] + p_cr); break;
    }
    Item it;
    it.key = static_cast<uint16_t>(key);
    it.cat = cat;
    it.pad = 0;
    it.ai = rec.ai;
    it.bi = rec.bi;
    it.aoff = rec.aoff;
    it.boff = rec.boff;
    it.ma = rec.ma;
    it.mb = rec.mb;
    it.slot = slot;
    if (item_pos < caps.items) {  // the item scratch holds caps.items
        items[item_pos] = it;
        // The execution records: items that write a bitmap at [0, caps.items),
        // those that write array or run values at caps.items + [0, caps.items),
        // each in key order.
        const uint32_t big_before = gbase[C_BB] + gbase[C_MX] + gbase[C_CB] + p_bb + p_mx + p_cb;
        const bool big = cat == CAT_BB || cat == CAT_MIXED || cat == CAT_COPY_BMP;
        const uint32_t r = big ? big_before : item_pos - big_before;
        if (r < caps.items) {  // (beyond it only when the plan overflows)
            ExecItem x;
            x.pos = static_cast<uint16_t>(item_pos);
            x.cat = cat;
            x.from_a = rec.ai >= 0 ? 1u : 0u;
            x.slot = slot;
            x.aoff = rec.aoff;
            x.boff = rec.boff;
            x.ma = rec.ma;
            x.mb = rec.mb;
            auto run0 = [](const uint16_t* runs, uint32_t meta, uint32_t off) -> uint32_t {
                if ((meta >> 16) != CR_RUN || (meta & 0xFFFFu) != 1u) return 0u;
                const uint16_t* r = runs + (off >> 1);
                return static_cast<uint32_t>(r[0]) | (static_cast<uint32_t>(r[1]) << 16);
            };
            x.run0_a = rec.ai >= 0 ? run0(run_a, rec.ma, rec.aoff) : 0u;
            x.run0_b = rec.bi >= 0 ? run0(run_b, rec.mb, rec.boff) : 0u;
            xitems[big ? r : caps.items + r] = x;
        }
    }
}

// ---- plan for two all-bitmap inputs with key indexes -------------------------
// Every pair is bitmap x bitmap and every one-sided key a bitmap copy, so a
// key's category follows from its presence in the two key_index arrays alone
// (an entry below n_containers).  One workgroup per 1024 keys; each first
// counts, over the whole key space with 16-byte loads, the items and pairs
// before its keys and in total (no workgroup waits on another), then ranks its
// own keys: item position in key order, bitmap slot with pairs first and
// copies after them, the reference's pool order (src/set_ops.cu:695-701).  The
// last workgroup writes the totals and flags an overflow when the key indexes
// do not name exactly n_containers keys per side or the plan outgrows the
// output capacity; an item whose container is not a bitmap is marked invalid
// (the compaction reports it).  Either way the host redoes the call on the
// exact path.
constexpr int KP_NT = 1024;

__device__ __forceinline__ uint64_t kidx_presence64(const uint16_t* kidx, uint32_t len, uint32_t n, uint32_t k0)
{
    uint64_t p = 0;
    if ((reinterpret_cast<uintptr_t>(kidx) & 15u) == 0 && k0 + 64u <= len) {
        const uint4* v = reinterpret_cast<const uint4*>(kidx + k0);
        uint4 x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = v[j];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t w[4] = {x[j].x, x[j].y, x[j].z, x[j].w};
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                p |= static_cast<uint64_t>((w[h] & 0xFFFFu) < n) << (8 * j + 2 * h);
                p |= static_cast<uint64_t>((w[h] >> 16) < n) << (8 * j + 2 * h + 1);
            }
        }
    } else {
        for (uint32_t k = 0; k < 64u && k0 + k < len; ++k) p |= static_cast<uint64_t>(kidx[k0 + k] < n) << k;
    }
    return p;
}

__global__ __launch_bounds__(KP_NT) void so_plan_bitmap(const uint16_t* __restrict__ kidx_a, uint32_t len_a,
                                                        const uint16_t* __restrict__ kidx_b, uint32_t len_b,
                                                        const uint32_t* __restrict__ off_a,
                                                        const uint32_t* __restrict__ off_b,
                                                        const uint8_t* __restrict__ ty_a,
                                                        const uint8_t* __restrict__ ty_b,
                                                        const uint16_t* __restrict__ cards_a,
                                                        const uint16_t* __restrict__ cards_b,
                                                        const uint16_t* __restrict__ keys_a,
                                                        const uint16_t* __restrict__ keys_b, uint32_t na, uint32_t nb,
                                                        uint32_t op, Caps caps, Item* items, Totals* totals,
                                                        uint32_t* kbad)
{
    __shared__ uint32_t lds[KP_NT / 64];
    const uint32_t t = threadIdx.x, g = blockIdx.x;
    const uint32_t kbase = g * KP_NT;
    auto item_mask = [op](uint64_t a, uint64_t b) {
        return op == CR_AND ? (a & b) : (op == CR_ANDNOT ? a : (a | b));
    };
    // Counts over the whole key space: thread t takes keys [64 t, 64 t + 64).
    const uint64_t pa = kidx_presence64(kidx_a, len_a, na, 64u * t);
    const uint64_t pb = kidx_presence64(kidx_b, len_b, nb, 64u * t);
    const uint64_t m = item_mask(pa, pb), mbb = m & pa & pb;
    // keys of this thread's 64 that lie before this workgroup's range
    const uint64_t before = 64u * t + 64u <= kbase ? ~0ull : (64u * t >= kbase ? 0ull : ((1ull << (kbase - 64u * t)) - 1ull));
    const uint32_t it_before = block_sum<KP_NT>(static_cast<uint32_t>(__popcll(m & before)), lds);
    const uint32_t bb_before = block_sum<KP_NT>(static_cast<uint32_t>(__popcll(mbb & before)), lds);
    const uint32_t bb_total = block_sum<KP_NT>(static_cast<uint32_t>(__popcll(mbb)), lds);
    // This workgroup's keys, one per thread.
    const uint32_t key = kbase + t;
    const uint32_t xa = key < len_a ? kidx_a[key] : 0xFFFFu;
    const uint32_t xb = key < len_b ? kidx_b[key] : 0xFFFFu;
    const bool ina = xa < na, inb = xb < nb;
    const bool is_item = (item_mask(ina, inb) & 1u) != 0;
    const bool is_bb = is_item && ina && inb;
    // Every named key must be the key its container holds; with the counts
    // checked below, the indexes then describe `keys` exactly.  The compaction
    // reads these per-workgroup counts (it runs after every workgroup here).
    const uint32_t bad = block_sum<KP_NT>((ina && keys_a[xa] != key) || (inb && keys_b[xb] != key) ? 1u : 0u, lds);
    if (t == 0) kbad[g] = bad;
    uint32_t n_here, bb_here, cb_here;
    const uint32_t r_item = block_flag_rank<KP_NT>(is_item, lds, n_here);
    const uint32_t r_bb = block_flag_rank<KP_NT>(is_bb, lds, bb_here);
    const uint32_t r_cb = block_flag_rank<KP_NT>(is_item && !is_bb, lds, cb_here);
    const uint32_t pos = it_before + r_item;
    if (is_item && pos < caps.items) {
        Item it;
        it.key = static_cast<uint16_t>(key);
        it.pad = 0;
        it.ai = ina ? static_cast<int32_t>(xa) : -1;
        it.bi = inb ? static_cast<int32_t>(xb) : -1;
        it.aoff = ina ? off_a[xa] : 0u;
        it.boff = inb ? off_b[xb] : 0u;
        // a container that is not a bitmap (counts that misdescribe the input)
        // makes the item invalid: the exec skips it and the compaction reports it
        const uint32_t ta = ina ? ty_a[xa] : 0u, tb = inb ? ty_b[xb] : 0u;
        it.ma = ina ? (ta << 16) | cards_a[xa] : 0u;
        it.mb = inb ? (tb << 16) | cards_b[xb] : 0u;
        const bool bitmaps = (!ina || ta == CR_BITMAP) && (!inb || tb == CR_BITMAP);
        it.cat = !bitmaps ? CAT_NONE : (is_bb ? CAT_BB : CAT_COPY_BMP);
        it.slot = is_bb ? bb_before + r_bb : bb_total + (it_before - bb_before) + r_cb;
        items[pos] = it;
    }
    if (g == gridDim.x - 1) {  // the last workgroup sees every key before its own
        const uint32_t n_items = it_before + n_here;
        const uint32_t n_a = block_sum<KP_NT>(static_cast<uint32_t>(__popcll(pa)), lds);
        const uint32_t n_b = block_sum<KP_NT>(static_cast<uint32_t>(__popcll(pb)), lds);
        if (t == 0) {
            for (int k = 0; k < C_N; ++k) totals->c[k] = 0;
            totals->c[C_ITEM] = n_items;
            totals->c[C_BB] = bb_total;
            totals->c[C_CB] = n_items - bb_total;
            totals->n_out = 0;
            totals->overflow = (n_a != na || n_b != nb || n_items > caps.items || n_items > caps.bmp) ? 1u : 0u;
        }
    }
}

// ---- execution: one wavefront per item --------------------------------------
// Every work item is a chain of dependent loads, and most are small, so the time
// follows the items in flight.  Each wave runs one item and exits, with no
// workgroup barrier, 20 waves a CU (8 KiB of LDS each); the grid covers the
// plan's bound and waves past the item count exit at once.  (A wave that went
// on to a second item would first wait for its stores: a wave's loads and
// stores retire in order.  Measured on the configs[2] pairs, that cost 5-15%.)
// The plan puts the containers' types and cards in the item, and writes the
// items in execution order -- bitmap-writing items first, the longest start
// first -- so a wave reads its record with one scalar load and then issues all
// its payload loads at once.  An 8 KiB bitmap is handled as eight 1 KiB pieces:
// lane l holds the 128-bit chunks l + 64 j (j < 8) of a side.
constexpr int EXEC_NT = 256;
constexpr uint32_t EXEC_LDS_WORDS = 2048;   // 8 KiB of LDS a wave
constexpr uint32_t EXEC_WAVES_PER_CU = 20;  // 160 KiB of LDS a CU

template <uint32_t OP>
__device__ __forceinline__ uint32_t apply32(uint32_t a, uint32_t b)
{
    if constexpr (OP == CR_AND) return a & b;
    if constexpr (OP == CR_OR) return a | b;
    if constexpr (OP == CR_ANDNOT) return a & ~b;
    return a ^ b;
}

template <uint32_t OP>
__device__ __forceinline__ uint4 apply4(const uint4& a, const uint4& b)
{
    return make_uint4(apply32<OP>(a.x, b.x), apply32<OP>(a.y, b.y), apply32<OP>(a.z, b.z), apply32<OP>(a.w, b.w));
}

__device__ __forceinline__ uint32_t popc4(const uint4& r) { return __popc(r.x) + __popc(r.y) + __popc(r.z) + __popc(r.w); }

__device__ __forceinline__ uint32_t uni(uint32_t v)
{
    return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
}

// The wave's total of v (DPP scan, no LDS addresses held in registers).
__device__ __forceinline__ uint32_t wave_total(uint32_t v)
{
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(wave_incl_scan(v)), 63));
}

__device__ __forceinline__ uint32_t lanes_below(uint64_t mask)
{
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
}

// A wave's record: the same for every lane, so it is read through the constant
// address space, one scalar load into scalar registers.
typedef uint32_t item_v8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ ExecItem load_xitem(const ExecItem* p)
{
    const item_v8 x = *reinterpret_cast<const __attribute__((address_space(4))) item_v8*>(reinterpret_cast<uintptr_t>(p));
    ExecItem it;
    it.pos = static_cast<uint16_t>(x[0]);
    it.cat = static_cast<uint8_t>(x[0] >> 16);
    it.from_a = static_cast<uint8_t>(x[0] >> 24);
    it.slot = x[1];
    it.aoff = x[2];
    it.boff = x[3];
    it.ma = x[4];
    it.mb = x[5];
    it.run0_a = x[6];
    it.run0_b = x[7];
    return it;
}

// A bitmap container's eight chunks of this lane.
__device__ __forceinline__ void bitmap_side(const uint64_t* pool, uint32_t off, uint32_t lane, uint4 (&c)[8])
{
    const uint32_t* src = reinterpret_cast<const uint32_t*>(pool) + (off >> 2);
    if ((off & 15u) == 0) {
#pragma unroll
        for (int j = 0; j < 8; ++j) c[j] = ld_stream(reinterpret_cast<const uint4*>(src) + lane + 64u * j);
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t* p = src + 4u * (lane + 64u * j);
            c[j] = make_uint4(p[0], p[1], p[2], p[3]);
        }
    }
}

__device__ __forceinline__ void zero_image(uint32_t* img, uint32_t lane)
{
#pragma unroll
    for (int j = 0; j < 8; ++j) reinterpret_cast<uint4*>(img)[lane + 64u * j] = make_uint4(0, 0, 0, 0);
    wave_lds_fence();
}

__device__ __forceinline__ void read_image(const uint32_t* img, uint32_t lane, uint4 (&c)[8])
{
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = reinterpret_cast<const uint4*>(img)[lane + 64u * j];
}

// The first payload words of a side, loaded for both sides as soon as the
// record is in, so that both sides' loads are in flight together: an array's
// values lane and lane + 64 (~0u past its end), or run `lane` as
// start | length << 16 and the run before it (0 for lane 0 or past the end).
// Bitmap and absent sides have none (a bitmap's 8 KiB are loaded whole).
struct Pre {
    uint32_t v0, v1;
};

__device__ __forceinline__ uint32_t run_word(const uint16_t* runs, uint32_t i, bool al4)
{
    if (al4) return reinterpret_cast<const uint32_t*>(runs)[i];
    return static_cast<uint32_t>(runs[2 * i]) | (static_cast<uint32_t>(runs[2 * i + 1]) << 16);
}

__device__ __forceinline__ bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

__device__ __forceinline__ Pre preload(const Side& S, uint32_t meta, uint32_t off, uint32_t lane, uint32_t run0)
{
    const uint32_t ty = meta >> 16, n = meta & 0xFFFFu;
    Pre p{~0u, ~0u};
    if (ty == CR_RUN && n == 1u) {  // the record holds the run: no load
        p.v0 = lane == 0 ? run0 : 0u;
        p.v1 = 0u;
        return p;
    }
    if (ty == CR_ARRAY) {  // (an absent side: meta 0, no values)
        const uint16_t* vals = S.arr + (off >> 1);
        if (lane < n) p.v0 = vals[lane];
        if (lane + 64u < n) p.v1 = vals[lane + 64u];
    } else if (ty == CR_RUN) {
        const uint16_t* runs = S.run + (off >> 1);
        const bool al4 = aligned4(runs);
        p.v0 = lane < n ? run_word(runs, lane, al4) : 0u;
        p.v1 = lane > 0 && lane < n ? run_word(runs, lane - 1u, al4) : 0u;
    }
    return p;
}

// An array's values set as bits in the wave's image (LDS atomics; the first
// 128 from the preload, then four loads a lane in flight).
__device__ __forceinline__ void set_array(const uint16_t* vals, uint32_t n, const Pre& pre, uint32_t lane, uint32_t* img)
{
    if (pre.v0 != ~0u) atomicOr(&img[pre.v0 >> 5], 1u << (pre.v0 & 31u));
    if (pre.v1 != ~0u) atomicOr(&img[pre.v1 >> 5], 1u << (pre.v1 & 31u));
    for (uint32_t i0 = lane + 128u; i0 < n; i0 += 4u * 64u) {
        uint32_t v[4];
#pragma unroll
        for (uint32_t k = 0; k < 4u; ++k) v[k] = i0 + 64u * k < n ? static_cast<uint32_t>(vals[i0 + 64u * k]) : ~0u;
#pragma unroll
        for (uint32_t k = 0; k < 4u; ++k)
            if (v[k] != ~0u) atomicOr(&img[v[k] >> 5], 1u << (v[k] & 31u));
    }
    wave_lds_fence();
}

// A side that is not a bitmap, set in the wave's 8 KiB image.  An array's
// values become bits (LDS atomics).  A run container's runs become toggles:
// each run flips its first bit and the bit after its last (XOR: a run that
// starts where the previous one ends continues it), and image_chunk turns
// them into bits.  Runs that are not sorted and disjoint (no well-formed
// container has them) are ORed in as bits instead, as the reference's
// expansion does (src/set_ops.cu:322-368), ends past 0xFFFF clamped.  The
// first values come from `pre`.  Returns true when the image holds toggles.
__device__ __forceinline__ bool build_image(const Side& S, uint32_t meta, uint32_t off, const Pre& pre,
                                            uint32_t lane, uint32_t* img)
{
    const uint32_t ty = meta >> 16, n = meta & 0xFFFFu;
    zero_image(img, lane);
    if (ty == CR_ARRAY) {
        set_array(S.arr + (off >> 1), n, pre, lane, img);
        return false;
    }
    if (ty != CR_RUN) return false;  // an empty image
    const uint16_t* runs = S.run + (off >> 1);
    const bool al4 = aligned4(runs);
    bool bad = false;
    auto toggle = [&](uint32_t i, uint32_t cw, uint32_t pw) {
        const uint32_t st = cw & 0xFFFFu, en = min(0xFFFFu, st + (cw >> 16));
        bad |= i > 0 && st <= min(0xFFFFu, (pw & 0xFFFFu) + (pw >> 16));
        atomicXor(&img[st >> 5], 1u << (st & 31u));
        if (en < 0xFFFFu) atomicXor(&img[(en + 1u) >> 5], 1u << ((en + 1u) & 31u));
    };
    if (lane < n) toggle(lane, pre.v0, pre.v1);
    for (uint32_t i0 = lane + 64u; i0 < n; i0 += 2u * 64u) {
        uint32_t cw[2], pw[2];
#pragma unroll
        for (uint32_t k = 0; k < 2u; ++k) {
            const uint32_t i = i0 + 64u * k;
            cw[k] = i < n ? run_word(runs, i, al4) : 0u;
            pw[k] = i < n ? run_word(runs, i - 1u, al4) : 0u;
        }
#pragma unroll
        for (uint32_t k = 0; k < 2u; ++k)
            if (i0 + 64u * k < n) toggle(i0 + 64u * k, cw[k], pw[k]);
    }
    wave_lds_fence();
    if (__ballot(bad) == 0ull) return true;
    // Each run's words ORed in, the wave's lanes across its words: 64 runs
    // loaded at a time, one lane each, then taken in turn.
    zero_image(img, lane);
    for (uint32_t r0 = 0; r0 < n; r0 += 64u) {
        const uint32_t r = r0 + lane;
        const uint32_t cw = r < n ? run_word(runs, r, al4) : 0u;
        const uint32_t st = cw & 0xFFFFu, en = min(0xFFFFu, st + (cw >> 16));
        const uint32_t m = min(64u, n - r0);
        for (uint32_t k = 0; k < m; ++k) {
            const uint32_t s0 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(st), k));
            const uint32_t e0 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(en), k));
            for (uint32_t w = (s0 >> 5) + lane; w <= (e0 >> 5); w += 64u)
                atomicOr(&img[w], bit_span(w == (s0 >> 5) ? s0 & 31u : 0u, w == (e0 >> 5) ? e0 & 31u : 31u));
        }
    }
    wave_lds_fence();
    return false;
}

// Chunk l + 64 j of an image, read in the order j = 0..7.  With toggles each
// 32-bit word is its own prefix XOR (five shifts) flipped by the parity of
// every toggle before it: the words before it in the lane's chunk, the lanes
// before it in group j (a ballot), and groups 0..j-1 (`carry`).  A group with
// no toggle (most of them: a run container holds a few runs) is all ones or
// all zeros.
__device__ __forceinline__ uint4 image_chunk(const uint32_t* img, uint32_t lane, uint32_t j, bool toggles,
                                             uint32_t& carry)
{
    const uint4 x = reinterpret_cast<const uint4*>(img)[lane + 64u * j];
    if (!toggles) return x;
    if (__ballot((x.x | x.y | x.z | x.w) != 0u) == 0ull) {  // no toggle in the group: all as before it
        const uint32_t f = 0u - carry;
        return make_uint4(f, f, f, f);
    }
    uint32_t w[4] = {x.x, x.y, x.z, x.w};
    uint32_t p = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t y = w[q];
        y ^= y << 1;
        y ^= y << 2;
        y ^= y << 4;
        y ^= y << 8;
        y ^= y << 16;
        w[q] = y;
        p ^= y >> 31;  // the word's parity
    }
    const uint64_t m = __ballot(p != 0u);
    uint32_t in = (lanes_below(m) & 1u) ^ carry;  // parity before this lane's chunk
    carry ^= static_cast<uint32_t>(__popcll(m)) & 1u;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t pw = w[q] >> 31;
        w[q] ^= 0u - in;
        in ^= pw;
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// A run container of at most RUN_DIRECT runs, decoded in registers from the
// preload (run r in lane r).  For each run, the lane's chunks strictly inside
// it are all ones, and its first and last chunk take masks computed once for
// the wave; chunk groups the run does not reach are skipped.  Any order or
// overlap of the runs gives the reference's expansion (src/set_ops.cu:322-368),
// ends past 0xFFFF clamped.
constexpr uint32_t RUN_DIRECT = 4;

__device__ __forceinline__ uint4 chunk_span(uint32_t lo, uint32_t hi)  // bits lo..hi of a chunk, lo <= hi < 128
{
    uint32_t w[4];
#pragma unroll
    for (uint32_t q = 0; q < 4u; ++q) {
        const uint32_t wl = 32u * q, wh = wl + 31u;
        w[q] = (lo <= wh && hi >= wl) ? bit_span(max(lo, wl) - wl, min(hi, wh) - wl) : 0u;
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ __forceinline__ void run_direct(const Pre& pre, uint32_t n, uint32_t lane, uint4 (&c)[8])
{
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = make_uint4(0, 0, 0, 0);
    for (uint32_t r = 0; r < n; ++r) {
        const uint32_t wd = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(pre.v0), r));
        const uint32_t st = wd & 0xFFFFu, en = min(0xFFFFu, st + (wd >> 16));
        const uint32_t cs = st >> 7, ce = en >> 7;  // its first and last chunk
        const uint4 ms = chunk_span(st & 127u, cs == ce ? en & 127u : 127u);
        const uint4 me = chunk_span(0u, en & 127u);
        const uint32_t js = cs >> 6, je = ce >> 6;  // the chunk groups of its ends
#pragma unroll
        for (uint32_t j = 0; j < 8u; ++j) {
            if (j < js || j > je) continue;  // the run misses chunk group j
            const uint32_t ch = lane + 64u * j;
            const uint32_t f = (ch > cs && ch < ce) ? ~0u : 0u;
            c[j].x |= f, c[j].y |= f, c[j].z |= f, c[j].w |= f;
            if (j == js) {
                const bool at = lane == (cs & 63u);
                c[j].x |= at ? ms.x : 0u, c[j].y |= at ? ms.y : 0u, c[j].z |= at ? ms.z : 0u, c[j].w |= at ? ms.w : 0u;
            }
            if (j == je && ce != cs) {
                const bool at = lane == (ce & 63u);
                c[j].x |= at ? me.x : 0u, c[j].y |= at ? me.y : 0u, c[j].z |= at ? me.z : 0u, c[j].w |= at ? me.w : 0u;
            }
        }
    }
}

// A side's registers without an image: a bitmap's chunks loaded, or a short
// run container decoded.
__device__ __forceinline__ void held_side(const Side& S, uint32_t meta, uint32_t off, const Pre& pre, uint32_t lane,
                                          uint4 (&c)[8])
{
    if ((meta >> 16) == CR_BITMAP)
        bitmap_side(S.bmp, off, lane, c);
    else
        run_direct(pre, meta & 0xFFFFu, lane, c);
}

// Writes OP of the held chunks `x` (side A when X_IS_A) and the image's
// chunks to the 8 KiB output slot; returns the lane's popcount.
template <uint32_t OP, bool X_IS_A>
__device__ __forceinline__ uint32_t store_with_image(const uint4 (&x)[8], const uint32_t* img, bool toggles,
                                                     uint32_t lane, uint4* dst)
{
    uint32_t carry = 0, pc = 0;
#pragma unroll
    for (uint32_t j = 0; j < 8u; ++j) {
        const uint4 y = image_chunk(img, lane, j, toggles, carry);
        const uint4 r = X_IS_A ? apply4<OP>(x[j], y) : apply4<OP>(y, x[j]);
        st_stream(dst + lane + 64u * j, r);
        pc += popc4(r);
    }
    return pc;
}

// n u16 values, four loads a lane in flight.
__device__ __forceinline__ void wave_copy16(uint16_t* dst, const uint16_t* src, uint32_t n, uint32_t lane)
{
    for (uint32_t i0 = lane; i0 < n; i0 += 4u * 64u) {
        uint16_t v[4];
#pragma unroll
        for (uint32_t k = 0; k < 4u; ++k) v[k] = i0 + 64u * k < n ? src[i0 + 64u * k] : uint16_t(0);
#pragma unroll
        for (uint32_t k = 0; k < 4u; ++k)
            if (i0 + 64u * k < n) dst[i0 + 64u * k] = v[k];
    }
}

// An item that writes a bitmap (BB, MIXED, COPY_BMP), run by one wave;
// returns its card | keep << 31.
template <uint32_t OP>
__device__ __forceinline__ uint32_t run_big(const Side& A, const Side& B, const ExecItem& it, const Pre& pa,
                                            const Pre& pb, uint32_t lane, uint32_t* img, uint64_t* out_bmp)
{
    const uint32_t ta = it.ma >> 16, tb = it.mb >> 16;
    uint32_t card = 0;
    bool keep = true;
    switch (it.cat) {
    case CAT_BB:
    case CAT_MIXED: {
        // A bitmap side, or a run container of a few runs, is held in
        // registers (a bitmap's loads in flight while the other side's image
        // is built); an array or a longer run container goes through the
        // wave's image.  With two images, A's chunks are read into registers
        // before B's image replaces them.
        uint4* dst = reinterpret_cast<uint4*>(out_bmp + it.slot * 1024ull);  // 8 KiB slots: 16-byte aligned
        uint32_t pc = 0;
        const bool ha = ta == CR_BITMAP || (ta == CR_RUN && (it.ma & 0xFFFFu) <= RUN_DIRECT);
        const bool hb = tb == CR_BITMAP || (tb == CR_RUN && (it.mb & 0xFFFFu) <= RUN_DIRECT);
        uint4 x[8];
        if (ha && hb) {
            uint4 y[8];
            held_side(A, it.ma, it.aoff, pa, lane, x);
            held_side(B, it.mb, it.boff, pb, lane, y);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint4 r = apply4<OP>(x[j], y[j]);
                st_stream(dst + lane + 64u * j, r);
                pc += popc4(r);
            }
        } else if (ha) {
            held_side(A, it.ma, it.aoff, pa, lane, x);
            const bool tg = build_image(B, it.mb, it.boff, pb, lane, img);
            pc = store_with_image<OP, true>(x, img, tg, lane, dst);
        } else if (hb) {
            held_side(B, it.mb, it.boff, pb, lane, x);
            const bool tg = build_image(A, it.ma, it.aoff, pa, lane, img);
            pc = store_with_image<OP, false>(x, img, tg, lane, dst);
        } else {
            bool tg = build_image(A, it.ma, it.aoff, pa, lane, img);
            uint32_t carry = 0;
#pragma unroll
            for (uint32_t j = 0; j < 8u; ++j) x[j] = image_chunk(img, lane, j, tg, carry);
            tg = build_image(B, it.mb, it.boff, pb, lane, img);  // its zeroing follows the reads above
            pc = store_with_image<OP, true>(x, img, tg, lane, dst);
        }
        pc = wave_total(pc);
        card = pc > 65535u ? 0u : pc;  // 65536 stored as 0 (src/set_ops.cu:179-180)
        keep = card != 0 || OP == CR_OR;
        break;
    }
    case CAT_COPY_BMP: {
        const bool from_a = it.from_a != 0;
        uint4 c[8];
        bitmap_side(from_a ? A.bmp : B.bmp, from_a ? it.aoff : it.boff, lane, c);
        uint4* dst = reinterpret_cast<uint4*>(out_bmp + it.slot * 1024ull);
#pragma unroll
        for (int j = 0; j < 8; ++j) st_stream(dst + lane + 64u * j, c[j]);
        card = (from_a ? it.ma : it.mb) & 0xFFFFu;
        break;
    }
    default: break;
    }
    return card | (keep ? 0x80000000u : 0u);
}

// An item that writes array or run values (BA, AA, COPY_ARR, COPY_RUN), run by
// one wave; returns its card | keep << 31.
template <uint32_t OP>
__device__ __forceinline__ uint32_t run_small(const Side& A, const Side& B, const ExecItem& it, const Pre& pa,
                                              const Pre& pb, uint32_t lane, uint32_t* img, uint16_t* out_arr,
                                              uint16_t* out_run)
{
    const uint32_t ta = it.ma >> 16;
    uint32_t card = 0;
    bool keep = true;
    switch (it.cat) {
    case CAT_BA: {
        // AND of a bitmap and an array: the array's values whose bit is set,
        // compacted in array order with ballots (the output is sorted).
        const bool bmp_is_a = ta == CR_BITMAP;
        const uint64_t* bm = bmp_is_a ? A.bmp + (it.aoff >> 3) : B.bmp + (it.boff >> 3);
        const uint16_t* arr = bmp_is_a ? B.arr + (it.boff >> 1) : A.arr + (it.aoff >> 1);
        const uint32_t n = (bmp_is_a ? it.mb : it.ma) & 0xFFFFu;
        const Pre pv = bmp_is_a ? pb : pa;
        uint16_t* out = out_arr + it.slot;
        for (uint32_t t0 = 0; t0 < n; t0 += 4u * 64u) {  // four values a lane in flight
            uint32_t v[4];
            bool p[4];
#pragma unroll
            for (uint32_t k = 0; k < 4u; ++k) {
                const uint32_t i = t0 + 64u * k + lane;
                const uint32_t x = (t0 == 0 && k < 2u) ? (k == 0 ? pv.v0 : pv.v1)
                                                        : (i < n ? static_cast<uint32_t>(arr[i]) : 0u);
                v[k] = i < n ? x : 0u;
            }
#pragma unroll
            for (uint32_t k = 0; k < 4u; ++k) {
                const uint32_t i = t0 + 64u * k + lane;
                p[k] = i < n && ((bm[v[k] >> 6] >> (v[k] & 63u)) & 1u) != 0u;
            }
#pragma unroll
            for (uint32_t k = 0; k < 4u; ++k) {
                const uint64_t mask = __ballot(p[k]);
                if (p[k]) out[card + lanes_below(mask)] = static_cast<uint16_t>(v[k]);
                card += static_cast<uint32_t>(__popcll(mask));
            }
        }
        keep = card != 0;
        break;
    }
    case CAT_AA: {
        // AND of two arrays: one side's values set in the wave's image, the
        // other side's probed against it in order and compacted with ballots
        // (the output is sorted).  The longer side goes into the image.
        // The image is clear on entry (the wave clears it before its first
        // item) and is cleared again on exit: the words this item set, or
        // the whole image after more than 128 values.
        const uint32_t nx = it.ma & 0xFFFFu, ny = it.mb & 0xFFFFu;
        const bool img_a = nx > ny;
        const Pre pi = img_a ? pa : pb;
        const uint32_t ni = img_a ? nx : ny;
        set_array(img_a ? A.arr + (it.aoff >> 1) : B.arr + (it.boff >> 1), ni, pi, lane, img);
        const uint16_t* vals = img_a ? B.arr + (it.boff >> 1) : A.arr + (it.aoff >> 1);
        const Pre pv = img_a ? pb : pa;
        const uint32_t n = img_a ? ny : nx;
        uint16_t* out = out_arr + it.slot;
        for (uint32_t t0 = 0; t0 < n; t0 += 64u) {
            const uint32_t i = t0 + lane;
            bool p = false;
            uint32_t v = 0;
            if (i < n) {
                v = t0 == 0 ? pv.v0 : (t0 == 64u ? pv.v1 : static_cast<uint32_t>(vals[i]));
                p = ((img[v >> 5] >> (v & 31u)) & 1u) != 0u;
            }
            const uint64_t mask = __ballot(p);
            if (p) out[card + lanes_below(mask)] = static_cast<uint16_t>(v);
            card += static_cast<uint32_t>(__popcll(mask));
        }
        wave_lds_fence();  // the probes are done before the image is cleared
        if (ni > 128u) {
            zero_image(img, lane);
        } else {
            if (pi.v0 != ~0u) img[pi.v0 >> 5] = 0u;
            if (pi.v1 != ~0u) img[pi.v1 >> 5] = 0u;
            wave_lds_fence();
        }
        keep = card != 0;
        break;
    }
    case CAT_COPY_ARR:
    case CAT_COPY_RUN: {
        // the first 128 values (64 runs) from the preload, the rest copied
        const bool from_a = it.from_a != 0;
        const Pre pv = from_a ? pa : pb;
        card = (from_a ? it.ma : it.mb) & 0xFFFFu;
        const uint16_t* src;
        uint16_t* dst;
        uint32_t n;
        if (it.cat == CAT_COPY_ARR) {
            src = (from_a ? A.arr : B.arr) + ((from_a ? it.aoff : it.boff) >> 1);
            dst = out_arr + it.slot;
            n = card;
            if (lane < n) dst[lane] = static_cast<uint16_t>(pv.v0);
            if (lane + 64u < n) dst[lane + 64u] = static_cast<uint16_t>(pv.v1);
        } else {
            src = (from_a ? A.run : B.run) + ((from_a ? it.aoff : it.boff) >> 1);
            dst = out_run + it.slot;
            n = 2u * card;
            if (lane < card) {
                dst[2u * lane] = static_cast<uint16_t>(pv.v0);
                dst[2u * lane + 1u] = static_cast<uint16_t>(pv.v0 >> 16);
            }
        }
        if (n > 128u) wave_copy16(dst + 128, src + 128, n - 128u, lane);
        break;
    }
    default: break;
    }
    return card | (keep ? 0x80000000u : 0u);
}

// Waves [0, n_big_waves) run the bitmap-writing items, one each (those past
// their count exit); the waves after them take SMALL_PER_WAVE of the other
// items each.  The plan wrote the records of the first kind at xitems[0, stride)
// and of the second at xitems[stride, 2 stride), so a wave's records sit at
// offsets known at launch and load in the same scalar-load round as the
// plan's totals.  A small-item wave loads
// all its records and first payload words, then waits for all of them once:
// from then on no item waits for an earlier one's stores (a wave's loads and
// stores retire in order, and the compiler cannot count stores issued in
// loops).
constexpr uint32_t SMALL_PER_WAVE = 4;

template <uint32_t OP>
__global__ __launch_bounds__(EXEC_NT) __attribute__((amdgpu_waves_per_eu(EXEC_WAVES_PER_CU / 4u))) void so_exec(
    Side A, Side B, const ExecItem* __restrict__ xitems, uint32_t stride, uint32_t n_big_waves, const Totals* totals,
    uint64_t* __restrict__ out_bmp, uint16_t* __restrict__ out_arr, uint16_t* __restrict__ out_run,
    uint32_t* __restrict__ item_card)
{
    __shared__ alignas(16) uint32_t lds[(EXEC_NT / 64) * EXEC_LDS_WORDS];
    const uint32_t w = uni((blockIdx.x * EXEC_NT + threadIdx.x) >> 6);
    const uint32_t lane = __lane_id();
    uint32_t* img = lds + (threadIdx.x >> 6) * EXEC_LDS_WORDS;
    if (w < n_big_waves) {
        const ExecItem it = load_xitem(xitems + min(w, stride - 1u));
        const uint32_t n_big = totals->c[C_BB] + totals->c[C_MX] + totals->c[C_CB];
        // (the output was not allocated for an overflowed plan)
        if (totals->overflow || w >= n_big) return;
        const Pre pa = preload(A, it.ma, it.aoff, lane, it.run0_a), pb = preload(B, it.mb, it.boff, lane, it.run0_b);
        const uint32_t r = run_big<OP>(A, B, it, pa, pb, lane, img, out_bmp);
        if (lane == 0) item_card[it.pos] = r;
        return;
    }
    const uint32_t first = SMALL_PER_WAVE * (w - n_big_waves);
    ExecItem it[SMALL_PER_WAVE];
#pragma unroll
    for (uint32_t k = 0; k < SMALL_PER_WAVE; ++k)
        if (first + k < stride) it[k] = load_xitem(xitems + stride + first + k);
    const uint32_t n_small = totals->c[C_ITEM] - (totals->c[C_BB] + totals->c[C_MX] + totals->c[C_CB]);
    if (totals->overflow || first >= n_small) return;
    const uint32_t cnt = min(SMALL_PER_WAVE, n_small - first);
    Pre pa[SMALL_PER_WAVE], pb[SMALL_PER_WAVE];
#pragma unroll
    for (uint32_t k = 0; k < SMALL_PER_WAVE; ++k)
        if (k < cnt) {
            pa[k] = preload(A, it[k].ma, it[k].aoff, lane, it[k].run0_a);
            pb[k] = preload(B, it[k].mb, it[k].boff, lane, it[k].run0_b);
        }
    zero_image(img, lane);  // array x array items keep it clear between them
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): every preload is in
#pragma unroll
    for (uint32_t k = 0; k < SMALL_PER_WAVE; ++k)
        if (k < cnt) {
            const uint32_t r = run_small<OP>(A, B, it[k], pa[k], pb[k], lane, img, out_arr, out_run);
            if (lane == 0) item_card[it[k].pos] = r;
        }
}

// item_card: bit 31 = keep, bit 30 = an invalid item (the plan found a
// container that is not a bitmap), low 16 bits = the stored card.
constexpr uint32_t ITEM_INVALID = 0x40000000u;

// ---- bitmap x bitmap only: one wavefront per pair ----------------------------
// When both inputs are all-bitmap every work item is a bitmap pair or a
// one-sided bitmap copy.  Each wave streams one item: for a pair 64 lanes x 8
// x 16-byte loads per input, all sixteen issued before the op, then the stores
// and a wave-level popcount; a copy moves one side's 8 KiB.  No workgroup
// barrier anywhere.
constexpr int BB_NT = 256;

template <uint32_t OP>
__global__ __launch_bounds__(BB_NT) void so_exec_bb(const uint64_t* __restrict__ a_bmp, const uint64_t* __restrict__ b_bmp,
                                                    const Item* __restrict__ items, const Totals* totals,
                                                    uint64_t* __restrict__ out_bmp, uint32_t* __restrict__ item_card)
{
    if (totals->overflow) return;  // the output was not allocated for this plan
    const uint32_t n_items = totals->c[C_ITEM];
    const uint32_t lane = __lane_id();
    const uint32_t n_waves = gridDim.x * (BB_NT / 64);
    uint32_t w = (blockIdx.x * BB_NT + threadIdx.x) >> 6;
    if (w >= n_items) return;
    Item it = items[w];
    for (; w < n_items; w += n_waves) {
        const Item cur = it;
        if (w + n_waves < n_items) it = items[w + n_waves];  // prefetch the next item's record
        const uint64_t* pa = a_bmp + (cur.aoff >> 3);
        const uint64_t* pb = b_bmp + (cur.boff >> 3);
        uint64_t* po = out_bmp + cur.slot * 1024ull;
        uint32_t pc = 0;
        if (cur.cat != CAT_BB && cur.cat != CAT_COPY_BMP) {  // invalid (not bitmaps): nothing read or written
            if (lane == 0) item_card[w] = ITEM_INVALID;
            continue;
        }
        if (cur.cat == CAT_COPY_BMP) {  // a one-sided key: its container and stored card copied, always kept
            const bool from_a = cur.ai >= 0;
            const uint64_t* src = from_a ? pa : pb;
            if (((from_a ? cur.aoff : cur.boff) & 15u) == 0) {
                uint4 x[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) x[k] = ld_stream(reinterpret_cast<const uint4*>(src) + lane + 64 * k);
#pragma unroll
                for (int k = 0; k < 8; ++k) st_stream(reinterpret_cast<uint4*>(po) + lane + 64 * k, x[k]);
            } else {
                for (uint32_t i = lane; i < 1024u; i += 64) po[i] = src[i];
            }
            if (lane == 0) item_card[w] = ((from_a ? cur.ma : cur.mb) & 0xFFFFu) | 0x80000000u;
            continue;
        }
        if (((cur.aoff | cur.boff) & 15u) == 0) {
            const uint4* a4 = reinterpret_cast<const uint4*>(pa);
            const uint4* b4 = reinterpret_cast<const uint4*>(pb);
            uint4* o4 = reinterpret_cast<uint4*>(po);
            uint4 x[8], y[8];  // all 16 loads of the pair in flight before any store
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                x[k] = ld_stream(a4 + lane + 64 * k);
                y[k] = ld_stream(b4 + lane + 64 * k);
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                uint4 r;
                r.x = apply32<OP>(x[k].x, y[k].x);
                r.y = apply32<OP>(x[k].y, y[k].y);
                r.z = apply32<OP>(x[k].z, y[k].z);
                r.w = apply32<OP>(x[k].w, y[k].w);
                st_stream(o4 + lane + 64 * k, r);
                pc += __popc(r.x) + __popc(r.y) + __popc(r.z) + __popc(r.w);
            }
        } else {
            for (uint32_t i = lane; i < 1024u; i += 64) {
                const uint64_t x = pa[i], y = pb[i];
                const uint64_t r =
                    static_cast<uint64_t>(apply32<OP>(static_cast<uint32_t>(x), static_cast<uint32_t>(y))) |
                    (static_cast<uint64_t>(apply32<OP>(static_cast<uint32_t>(x >> 32), static_cast<uint32_t>(y >> 32)))
                     << 32);
                po[i] = r;
                pc += __popcll(r);
            }
        }
        pc = wave_sum(pc);
        if (lane == 0) {
            const uint32_t card = pc > 65535u ? 0u : pc;  // 65536 stored as 0 (src/set_ops.cu:179-180)
            const bool keep = card != 0 || OP == CR_OR;
            item_card[w] = card | (keep ? 0x80000000u : 0u);
        }
    }
}

// ---- two dense all-bitmap inputs: no plan -------------------------------------
// When both inputs hold a bitmap for every key of [0, n) (n_containers ==
// max_key + 1 with sorted unique keys, so container i has key i), pair i is
// key i on both sides, its output slot is i, and there is nothing to plan.
// One wave per pair, as so_exec_bb; cards go to item_card for the compaction.
template <uint32_t OP>
__global__ __launch_bounds__(BB_NT) void so_exec_dense(const uint64_t* __restrict__ a_bmp,
                                                       const uint64_t* __restrict__ b_bmp,
                                                       const uint32_t* __restrict__ off_a,
                                                       const uint32_t* __restrict__ off_b, uint32_t n,
                                                       uint64_t* __restrict__ out_bmp, uint32_t* __restrict__ item_card)
{
    const uint32_t lane = __lane_id();
    const uint32_t w = (blockIdx.x * BB_NT + threadIdx.x) >> 6;
    if (w >= n) return;
    const uint32_t oa = off_a[w], ob = off_b[w];
    const uint64_t* pa = a_bmp + (oa >> 3);
    const uint64_t* pb = b_bmp + (ob >> 3);
    uint64_t* po = out_bmp + static_cast<uint64_t>(w) * 1024u;
    uint32_t pc = 0;
    if (((oa | ob) & 15u) == 0) {
        const uint4* a4 = reinterpret_cast<const uint4*>(pa);
        const uint4* b4 = reinterpret_cast<const uint4*>(pb);
        uint4* o4 = reinterpret_cast<uint4*>(po);
        uint4 x[8], y[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            x[k] = ld_stream(a4 + lane + 64 * k);
            y[k] = ld_stream(b4 + lane + 64 * k);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            uint4 r;
            r.x = apply32<OP>(x[k].x, y[k].x);
            r.y = apply32<OP>(x[k].y, y[k].y);
            r.z = apply32<OP>(x[k].z, y[k].z);
            r.w = apply32<OP>(x[k].w, y[k].w);
            st_stream(o4 + lane + 64 * k, r);
            pc += __popc(r.x) + __popc(r.y) + __popc(r.z) + __popc(r.w);
        }
    } else {
        for (uint32_t i = lane; i < 1024u; i += 64) {
            const uint64_t x = pa[i], y = pb[i];
            const uint64_t r = static_cast<uint64_t>(apply32<OP>(static_cast<uint32_t>(x), static_cast<uint32_t>(y))) |
                               (static_cast<uint64_t>(apply32<OP>(static_cast<uint32_t>(x >> 32),
                                                                  static_cast<uint32_t>(y >> 32)))
                                << 32);
            po[i] = r;
            pc += __popcll(r);
        }
    }
    pc = wave_sum(pc);
    if (lane == 0) {
        const uint32_t card = pc > 65535u ? 0u : pc;  // 65536 stored as 0 (src/set_ops.cu:179-180)
        const bool keep = card != 0 || OP == CR_OR;
        item_card[w] = card | (keep ? 0x80000000u : 0u);
    }
}

// Compaction of the dense path: item i is key i in bitmap slot i.  One
// workgroup per 1024 items, each counting the kept items before it; the last
// writes the totals (every item a bitmap pair) into the pinned host slot.
__global__ __launch_bounds__(PLAN_NT) void so_compact_dense(const uint32_t* item_card, uint32_t n, uint16_t* keys,
                                                            uint8_t* types, uint32_t* offsets, uint16_t* cards,
                                                            SetOpHost* host)
{
    __shared__ uint32_t lds[PLAN_NT / 64];
    const uint32_t tile = blockIdx.x, t = threadIdx.x;
    uint32_t b = 0;
    for (uint32_t i = t; i < tile * PLAN_NT; i += PLAN_NT) b += item_card[i] >> 31;
    const uint32_t base = block_sum<PLAN_NT>(b, lds);
    const uint32_t w = tile * PLAN_NT + t;
    const uint32_t c = w < n ? item_card[w] : 0u;
    const bool keep = (c & 0x80000000u) != 0;
    uint32_t tot;
    const uint32_t r = block_flag_rank<PLAN_NT>(keep, lds, tot);
    if (keep) {
        const uint32_t o = base + r;
        keys[o] = static_cast<uint16_t>(w);
        types[o] = CR_BITMAP;
        offsets[o] = w * 8192u;
        cards[o] = static_cast<uint16_t>(c & 0xFFFFu);
    }
    if ((tile + 1) * PLAN_NT >= n && t < 64) {
        volatile uint32_t* h = reinterpret_cast<volatile uint32_t*>(host);
        if (t < C_N) h[t] = t == C_ITEM || t == C_BB ? n : 0u;
        if (t == C_N) h[C_N] = base + tot;
        if (t == C_N + 1) h[C_N + 1] = 0u;
    }
}

// ---- compaction of the kept containers -------------------------------------
// Lanes 0 .. C_N + 1 of a wave each write one field, so the posted writes to
// host memory go out together.
__device__ void write_host_totals(const Totals* totals, uint32_t n_out, uint32_t overflow, SetOpHost* host,
                                  uint32_t lane)
{
    volatile uint32_t* h = reinterpret_cast<volatile uint32_t*>(host);
    if (lane < C_N) h[lane] = totals->c[lane];
    if (lane == C_N) h[C_N] = n_out;
    if (lane == C_N + 1) h[C_N + 1] = overflow;
}

// The last tile's workgroup writes the kept count (and, given `host`, every
// total into the pinned slot); with no items or an overflowed plan workgroup 0
// does, and nothing is compacted.
__global__ __launch_bounds__(PLAN_NT) void so_compact(const Item* items, const uint32_t* item_card,
                                                      Totals* totals, uint16_t* keys,
                                                      uint8_t* types, uint32_t* offsets, uint16_t* cards,
                                                      SetOpHost* host, const uint32_t* kbad, uint32_t n_kbad)
{
    __shared__ uint32_t lds[PLAN_NT / 64];
    __shared__ uint32_t s_base;
    const uint32_t n_items = totals->c[C_ITEM];
    const uint32_t tile = blockIdx.x;
    // The key-index plan's check of its named keys (n_kbad <= 64 workgroups):
    // a mismatch invalidates the plan like an overflow.
    // Each wave reads all the counts itself, so every wave decides alike.
    uint32_t kb = 0;
    if (n_kbad) {
        const uint32_t lane = __lane_id();
        kb = __ballot(lane < min(n_kbad, 64u) && kbad[lane] != 0u) != 0ull ? 1u : 0u;
    }
    const uint32_t overflow = totals->overflow | kb;
    if (overflow || n_items == 0) {
        if (tile == 0 && threadIdx.x < 64 && host) write_host_totals(totals, 0, overflow, host, threadIdx.x);
        return;
    }
    if (tile * PLAN_NT >= n_items) return;
    const uint32_t t = threadIdx.x;
    const bool last = (tile + 1) * PLAN_NT >= n_items;
    uint32_t invalid = 0;
    {  // kept items before this tile, counted cooperatively (the last tile also counts invalid ones):
       // 16-byte loads of the cards (whole tiles of PLAN_NT, 256-byte aligned), four in flight a thread
        uint32_t b = 0;
        const uint4* c4 = reinterpret_cast<const uint4*>(item_card);
        const uint32_t n4 = tile * (PLAN_NT / 4);
        for (uint32_t i0 = t; i0 < n4; i0 += 4u * PLAN_NT) {
            uint4 x[4];
#pragma unroll
            for (uint32_t k = 0; k < 4u; ++k) {
                const uint32_t j = i0 + k * PLAN_NT;
                x[k] = j < n4 ? c4[j] : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (uint32_t k = 0; k < 4u; ++k) {
                b += (x[k].x >> 31) + (x[k].y >> 31) + (x[k].z >> 31) + (x[k].w >> 31);
                invalid += ((x[k].x >> 30) & 1u) + ((x[k].y >> 30) & 1u) + ((x[k].z >> 30) & 1u) + ((x[k].w >> 30) & 1u);
            }
        }
        b = block_sum<PLAN_NT>(b, lds);
        if (t == 0) s_base = b;
    }
    const uint32_t w = tile * PLAN_NT + t;
    bool keep = false;
    uint32_t c = 0;
    Item it{};
    if (w < n_items) {
        c = item_card[w];
        keep = (c & 0x80000000u) != 0;
        invalid += (c >> 30) & 1u;
        it = items[w];
    }
    if (last) invalid = block_sum<PLAN_NT>(invalid, lds);
    uint32_t tot;
    const uint32_t r = block_flag_rank<PLAN_NT>(keep, lds, tot);
    const uint32_t base = s_base;
    if (keep) {
        const uint32_t o = base + r;
        keys[o] = it.key;
        uint8_t ty;
        uint32_t off;
        switch (it.cat) {
        case CAT_BB:
        case CAT_MIXED:
        case CAT_COPY_BMP:
            ty = CR_BITMAP;
            off = it.slot * 8192u;
            break;
        case CAT_COPY_RUN:
            ty = CR_RUN;
            off = it.slot * 2u;
            break;
        default:
            ty = CR_ARRAY;
            off = it.slot * 2u;
            break;
        }
        types[o] = ty;
        offsets[o] = off;
        cards[o] = static_cast<uint16_t>(c & 0xFFFFu);
    }
    if (t < 64 && last) {
        if (t == 0) totals->n_out = base + tot;
        if (host) write_host_totals(totals, base + tot, invalid ? 1u : 0u, host, t);
    }
}

// DeMorgan rewrite (src/set_ops.cu:533-565).
static void resolve_negation(uint32_t& op, const cr_gpu_roaring*& a, const cr_gpu_roaring*& b, bool& neg)
{
    const bool na = a->negated, nb = b->negated;
    neg = false;
    if (!na && !nb) return;
    switch (op) {
    case CR_AND:
        if (na && !nb) {
            op = CR_ANDNOT;
            std::swap(a, b);
        } else if (!na && nb) {
            op = CR_ANDNOT;
        } else {
            op = CR_OR;
            neg = true;
        }
        break;
    case CR_OR:
        if (na && !nb) {
            op = CR_ANDNOT;
            neg = true;
        } else if (!na && nb) {
            op = CR_ANDNOT;
            std::swap(a, b);
            neg = true;
        } else {
            op = CR_AND;
            neg = true;
        }
        break;
    case CR_ANDNOT:
        if (na && !nb) {
            op = CR_OR;
            neg = true;
        } else if (!na && nb) {
            op = CR_AND;
        } else {
            op = CR_ANDNOT;
            std::swap(a, b);
        }
        break;
    default:  // XOR
        neg = !(na && nb);
        break;
    }
}

static unsigned exec_grid(uint32_t n_items)
{
    const uint32_t cus = num_cus();
    const uint32_t cap = static_cast<uint32_t>(cus) * 8u;  // 8 workgroups of 4 waves per CU
    return std::max(1u, std::min(n_items, cap));
}

// Output capacity known on the host before planning, from the inputs'
// container counts by type (src/set_ops.cu:626-692 fixes which pair gives
// which output type):
//   AND     bitmaps: pairs of two non-array containers, or a run and an array;
//           arrays: bitmap x array keeps the array side's values, array x
//           array at most the smaller side's -- both within the inputs' array
//           pools; no runs;
//   OR/XOR  every matched pair gives a bitmap, one-sided keys copy their
//           container: bitmaps <= m + min(bmp_a, na - m) + min(bmp_b, nb - m)
//           over the unknown number m of matched keys; arrays and runs <= the
//           inputs' pools;
//   ANDNOT  as OR with only A's one-sided keys copied.
// For inputs whose counts describe their containers (every upload, and
// set-operation results, whose counts include dropped slots) the plan fits;
// the plan kernel checks it anyway, and a plan that does not fit is redone by
// the exact two-pass path.
static Caps setop_caps(const cr_gpu_roaring* a, const cr_gpu_roaring* b, uint32_t op, uint32_t bound)
{
    const uint64_t na = a->n_containers, nb = b->n_containers;
    const uint64_t ba = a->n_bitmap_containers, bb = b->n_bitmap_containers;
    const uint64_t ra = a->n_run_containers, rb = b->n_run_containers;
    const uint64_t aa = a->n_array_containers, ab = b->n_array_containers;
    const uint64_t ea = a->array_pool_bytes / 2u, eb = b->array_pool_bytes / 2u;
    const uint64_t pa = a->run_pool_bytes / 2u, pb = b->run_pool_bytes / 2u;  // u16 entries
    const uint64_t m_max = std::min(na, nb);
    uint64_t bmp = 0, arr = 0, run = 0;
    auto clampm = [&](int64_t m) { return static_cast<uint64_t>(std::max<int64_t>(0, std::min<int64_t>(m, m_max))); };
    if (op == CR_AND) {
        bmp = std::min(ba + ra, bb + rb) + std::min(ra, ab) + std::min(aa, rb);
        bmp = std::min(bmp, m_max);
        arr = ea + eb;
    } else if (op == CR_ANDNOT) {
        for (int64_t m : {int64_t(0), int64_t(m_max), int64_t(na) - int64_t(ba)}) {
            const uint64_t mm = clampm(m);
            bmp = std::max(bmp, mm + std::min(ba, na - mm));
        }
        arr = ea;
        run = pa;
    } else {
        for (int64_t m : {int64_t(0), int64_t(m_max), int64_t(na) - int64_t(ba), int64_t(nb) - int64_t(bb)}) {
            const uint64_t mm = clampm(m);
            bmp = std::max(bmp, mm + std::min(ba, na - mm) + std::min(bb, nb - mm));
        }
        arr = ea + eb;
        run = pa + pb;
    }
    auto c32 = [](uint64_t x) { return static_cast<uint32_t>(std::min<uint64_t>(x, 0xFFFFFFFFull)); };
    Caps caps{bound, c32(std::min<uint64_t>(bmp, bound)), c32(arr), c32(run), 0u};
    // Each item that writes array or run values takes at least one array or run
    // container: for AND only an array (bitmap x array or array x array), for
    // ANDNOT one of A's (a copy of an A-only key, or an A array against B).
    const uint64_t small = op == CR_AND ? aa + ab : (op == CR_ANDNOT ? aa + ra : aa + ra + ab + rb);
    caps.small = c32(std::min<uint64_t>(bound, small));
    return caps;
}

// The plan (classify + assign) for `bound` work items into fresh scratch.
struct SetOpPlan {
    Scratch sc;
    Item* items;
    ExecItem* xitems = nullptr;  // so_plan_assign: bitmap-writing items, then (from `xstride`) the others
    uint32_t xstride = 0;       // the plan's bound
    Totals* tot;
    uint32_t* icard;
    uint32_t n_tiles;
    uint32_t* kbad = nullptr;  // key-index plan: per-workgroup counts of mismatched named keys
    uint32_t n_kbad = 0;
};

static int plan_set_operation(const Side& A, const Side& B, uint32_t op, uint32_t bound, const Caps& caps,
                              hipStream_t s, SetOpPlan& P)
{
    P.n_tiles = (bound + PLAN_NT - 1) / PLAN_NT;
    Carver c;
    const size_t o_recs = c.add(sizeof(KeyRec) * 65536);
    const size_t o_gc = c.add(sizeof(uint32_t) * PLAN_GROUPS * C_N);
    const size_t o_items = c.add(sizeof(Item) * bound);
    const size_t o_xitems = c.add(sizeof(ExecItem) * 2u * bound);
    const size_t o_tot = c.add(sizeof(Totals));
    const size_t o_card = c.add(sizeof(uint32_t) * bound);
    CR_RET(P.sc.alloc(c.total, s));
    KeyRec* recs = P.sc.at<KeyRec>(o_recs);
    uint32_t* gc = P.sc.at<uint32_t>(o_gc);
    P.items = P.sc.at<Item>(o_items);
    P.xitems = P.sc.at<ExecItem>(o_xitems);
    P.xstride = bound;  // = caps.items, where so_plan_assign starts the second kind
    P.tot = P.sc.at<Totals>(o_tot);
    P.icard = P.sc.at<uint32_t>(o_card);
    {
        CR_TIMED("so_plan_classify", s);
        so_plan_classify<<<PLAN_GROUPS, PLAN_NT, 0, s>>>(A, B, op, recs, gc);
    }
    CR_LAUNCH_CHECK();
    {
        CR_TIMED("so_plan_assign", s);
        so_plan_assign<<<PLAN_GROUPS, PLAN_NT, 0, s>>>(recs, gc, P.items, P.xitems, P.tot, caps, A.run, B.run);
    }
    CR_LAUNCH_CHECK();
    return CR_OK;
}

// The key-index plan of two all-bitmap inputs (so_plan_bitmap).
static int plan_bitmap_keyed(const cr_gpu_roaring* a, const cr_gpu_roaring* b, uint32_t op, uint32_t bound,
                             const Caps& caps, hipStream_t s, SetOpPlan& P)
{
    P.n_tiles = (bound + PLAN_NT - 1) / PLAN_NT;
    Carver c;
    const size_t o_items = c.add(sizeof(Item) * bound);
    const size_t o_tot = c.add(sizeof(Totals));
    const size_t o_card = c.add(sizeof(uint32_t) * bound);
    const size_t o_bad = c.add(sizeof(uint32_t) * 64);
    CR_RET(P.sc.alloc(c.total, s));
    P.items = P.sc.at<Item>(o_items);
    P.tot = P.sc.at<Totals>(o_tot);
    P.icard = P.sc.at<uint32_t>(o_card);
    P.kbad = P.sc.at<uint32_t>(o_bad);
    {
        CR_TIMED("so_plan_bitmap", s);
        const uint32_t len_a = a->max_key + 1u, len_b = b->max_key + 1u;
        const uint32_t groups = (std::max(len_a, len_b) + KP_NT - 1) / KP_NT;  // max_key <= 0xFFFF: <= 64
        P.n_kbad = groups;
        so_plan_bitmap<<<groups, KP_NT, 0, s>>>(a->key_index, len_a, b->key_index, len_b, a->offsets, b->offsets,
                                                a->types, b->types, a->cardinalities, b->cardinalities,
                                                a->keys, b->keys, a->n_containers,
                                                b->n_containers, op, caps, P.items, P.tot, P.kbad);
    }
    CR_LAUNCH_CHECK();
    return CR_OK;
}

// Execution and compaction of a plan into `out` (allocated for at most
// `bound` items); `host` (optional) receives the totals.
static int exec_set_operation(const Side& A, const Side& B, uint32_t op, uint32_t bound, uint32_t big_max,
                              uint32_t small_max, bool only_bb,
                              const SetOpPlan& P, cr_gpu_roaring* out, SetOpHost* host, hipStream_t s)
{
    if (only_bb) {
        // One item per wave: every pair's 16 loads are in flight at once
        // (capping the grid at the resident waves, two pairs a wave, measured
        // 1.5% slower at 16384 pairs).  Waves past the plan's item count exit.
        const unsigned gb = std::max(1u, (bound + 3) / 4);
        CR_TIMED("so_exec", s);
        switch (op) {
        case CR_AND:
            so_exec_bb<CR_AND><<<gb, BB_NT, 0, s>>>(A.bmp, B.bmp, P.items, P.tot, out->bitmap_data,
                                                    P.icard);
            break;
        case CR_OR:
            so_exec_bb<CR_OR><<<gb, BB_NT, 0, s>>>(A.bmp, B.bmp, P.items, P.tot, out->bitmap_data,
                                                   P.icard);
            break;
        case CR_ANDNOT:
            so_exec_bb<CR_ANDNOT><<<gb, BB_NT, 0, s>>>(A.bmp, B.bmp, P.items, P.tot,
                                                       out->bitmap_data, P.icard);
            break;
        default:
            so_exec_bb<CR_XOR><<<gb, BB_NT, 0, s>>>(A.bmp, B.bmp, P.items, P.tot, out->bitmap_data,
                                                    P.icard);
            break;
        }
    } else {
        // a wave per bitmap-writing item, then one per SMALL_PER_WAVE others
        // (at most big_max and small_max of them: the plan flags more)
        const uint32_t waves = big_max + (small_max + SMALL_PER_WAVE - 1u) / SMALL_PER_WAVE;
        const unsigned g = std::max(1u, (waves + 3u) / 4u);
        CR_TIMED("so_exec", s);
        switch (op) {
        case CR_AND:
            so_exec<CR_AND><<<g, EXEC_NT, 0, s>>>(A, B, P.xitems, P.xstride, big_max, P.tot, out->bitmap_data, out->array_data,
                                                  out->run_data, P.icard);
            break;
        case CR_OR:
            so_exec<CR_OR><<<g, EXEC_NT, 0, s>>>(A, B, P.xitems, P.xstride, big_max, P.tot, out->bitmap_data, out->array_data,
                                                 out->run_data, P.icard);
            break;
        case CR_ANDNOT:
            so_exec<CR_ANDNOT><<<g, EXEC_NT, 0, s>>>(A, B, P.xitems, P.xstride, big_max, P.tot, out->bitmap_data,
                                                     out->array_data, out->run_data, P.icard);
            break;
        default:
            so_exec<CR_XOR><<<g, EXEC_NT, 0, s>>>(A, B, P.xitems, P.xstride, big_max, P.tot, out->bitmap_data, out->array_data,
                                                  out->run_data, P.icard);
            break;
        }
    }
    CR_LAUNCH_CHECK();
    {
        CR_TIMED("so_compact", s);
        so_compact<<<std::max(1u, P.n_tiles), PLAN_NT, 0, s>>>(P.items, P.icard, P.tot, out->keys,
                                                               out->types, out->offsets, out->cardinalities, host,
                                                               P.kbad, P.n_kbad);
    }
    CR_LAUNCH_CHECK();
    return CR_OK;
}

static void set_counts(cr_gpu_roaring* out, const uint32_t* c)
{
    out->n_bitmap_containers = c[C_BB] + c[C_MX] + c[C_CB];
    out->n_array_containers = c[C_BA] + c[C_AA] + c[C_CA];
    out->n_run_containers = c[C_CR];
    out->array_pool_bytes = (c[C_BAE] + c[C_AAE] + c[C_CAE]) * 2u;
    out->run_pool_bytes = c[C_CRP] * 4u;
}

// The exact path: plan, read the totals back (first sync), allocate the output
// exactly, execute, compact, read the kept count (second sync).
static bool aligned_bitmaps(const cr_gpu_roaring* a, const cr_gpu_roaring* b)
{
    return ((reinterpret_cast<uintptr_t>(a->bitmap_data) | reinterpret_cast<uintptr_t>(b->bitmap_data)) & 15u) == 0;
}

static int set_operation_exact(const cr_gpu_roaring* a, const cr_gpu_roaring* b, const Side& A, const Side& B,
                               uint32_t op, uint32_t bound, hipStream_t s, cr_gpu_roaring* out)
{
    SetOpPlan P;
    // Matched on `keys` (a key search, not the key indexes, which this path
    // does not trust), with room for `bound` items: with sorted keys each
    // container yields at most one item, so more means malformed input.
    Side As = A, Bs = B;
    As.kidx = Bs.kidx = nullptr;
    As.kidx_n = Bs.kidx_n = 0;
    const Caps unbounded{bound, 0xFFFFFFFFu, 0xFFFFFFFFu, 0xFFFFFFFFu, 0u, 0u, 0u, 0u, 0xFFFFFFFFu};
    CR_RET(plan_set_operation(As, Bs, op, bound, unbounded, s, P));
    Totals h{};
    CR_RET(read_back(&h, P.tot, sizeof(Totals), s));
    if (h.overflow) {
        set_error("set_operation: an input's keys name more containers than it holds");
        return CR_ERR_INVALID;
    }
    const uint32_t n_items = h.c[C_ITEM];
    if (n_items == 0) return CR_OK;
    const uint64_t n_bmp = static_cast<uint64_t>(h.c[C_BB]) + h.c[C_MX] + h.c[C_CB];
    const uint64_t arr_elems = static_cast<uint64_t>(h.c[C_BAE]) + h.c[C_AAE] + h.c[C_CAE];
    const uint64_t run_u16 = 2ull * h.c[C_CRP];
    const OutLayout L = plan_out(n_items, 0, n_bmp * 1024, arr_elems, run_u16);
    CR_RET(alloc_out(out, L, n_items, 0, n_bmp * 1024, arr_elems, run_u16, s));
    set_counts(out, h.c);
    const bool only_bb = h.c[C_BB] + h.c[C_CB] == n_items && aligned_bitmaps(a, b);
    CR_RET(exec_set_operation(As, Bs, op, n_items, n_items, n_items, only_bb, P, out, nullptr, s));
    uint32_t n_out = 0;
    CR_RET(read_back(&n_out, &P.tot->n_out, sizeof(uint32_t), s));
    out->n_containers = n_out;
    return CR_OK;
}

// Both inputs hold a bitmap for every key of [0, n): pair i is key i, no plan.
// One synchronisation; the output is allocated exactly (n bitmap slots).
static int set_operation_dense(const cr_gpu_roaring* a, const cr_gpu_roaring* b, uint32_t op, hipStream_t s,
                               cr_gpu_roaring* out)
{
    const uint32_t n = a->n_containers;
    const OutLayout L = plan_out(n, 0, static_cast<uint64_t>(n) * 1024u, 0, 0);
    CR_RET(alloc_out(out, L, n, 0, static_cast<uint64_t>(n) * 1024u, 0, 0, s));
    HostSlotGuard hs;
    CR_RET(hs.acquire());
    {
        Scratch sc;
        CR_RET(sc.alloc(sizeof(uint32_t) * n, s));
        uint32_t* icard = sc.at<uint32_t>(0);
        const unsigned gb = (n + 3) / 4;
        {
            CR_TIMED("so_exec", s);
            switch (op) {
            case CR_AND:
                so_exec_dense<CR_AND><<<gb, BB_NT, 0, s>>>(a->bitmap_data, b->bitmap_data, a->offsets, b->offsets, n,
                                                           out->bitmap_data, icard);
                break;
            case CR_OR:
                so_exec_dense<CR_OR><<<gb, BB_NT, 0, s>>>(a->bitmap_data, b->bitmap_data, a->offsets, b->offsets, n,
                                                          out->bitmap_data, icard);
                break;
            case CR_ANDNOT:
                so_exec_dense<CR_ANDNOT><<<gb, BB_NT, 0, s>>>(a->bitmap_data, b->bitmap_data, a->offsets, b->offsets,
                                                              n, out->bitmap_data, icard);
                break;
            default:
                so_exec_dense<CR_XOR><<<gb, BB_NT, 0, s>>>(a->bitmap_data, b->bitmap_data, a->offsets, b->offsets, n,
                                                           out->bitmap_data, icard);
                break;
            }
        }
        CR_LAUNCH_CHECK();
        {
            CR_TIMED("so_compact", s);
            so_compact_dense<<<(n + PLAN_NT - 1) / PLAN_NT, PLAN_NT, 0, s>>>(icard, n, out->keys, out->types,
                                                                             out->offsets, out->cardinalities,
                                                                             hs.dev<SetOpHost>());
        }
        CR_LAUNCH_CHECK();
        CR_RET(sync_stream(s));
    }
    const uint32_t n_out = hs.host<SetOpHost>()->n_out;
    out->n_bitmap_containers = n;  // allocated slots, dropped ones included (src/set_ops.cu:695-701)
    out->n_containers = n_out;
    return CR_OK;
}

int set_operation_impl(const cr_gpu_roaring* a, const cr_gpu_roaring* b, uint32_t op, hipStream_t s,
                       cr_gpu_roaring* out)
{
    bool neg = false;
    resolve_negation(op, a, b, neg);
    reset(out);
    out->universe_size = std::max(a->universe_size, b->universe_size);
    out->negated = neg;
    const uint32_t na = a->n_containers, nb = b->n_containers;
    uint32_t bound = op == CR_AND ? std::min(na, nb) : (op == CR_ANDNOT ? na : na + nb);
    if (bound == 0) return CR_OK;  // empty work list (src/set_ops.cu:588-593)
    const Side A = side_of(a), B = side_of(b);

    // One synchronisation: the output is allocated before planning, at the
    // capacity the inputs' counts bound; the compaction writes the totals into
    // a pinned host slot.
    Caps caps = setop_caps(a, b, op, bound);
    // Both inputs all-bitmap: every item is a bitmap pair or a bitmap copy (the
    // plan verifies it), and one wave streams each.
    const bool only_bb = a->n_array_containers == 0 && a->n_run_containers == 0 && b->n_array_containers == 0 &&
                         b->n_run_containers == 0 && aligned_bitmaps(a, b);
    if (only_bb && a->key_index && b->key_index && a->max_key == b->max_key && na == a->max_key + 1u &&
        nb == na && a->n_bitmap_containers == na && b->n_bitmap_containers == nb)
        return set_operation_dense(a, b, op, s, out);
    caps.bb_only = only_bb ? 1u : 0u;
    if (use_kidx(A.kidx, A.n, B.kidx, B.n)) {
        caps.check_kidx = 1u;
        caps.na = na;
        caps.nb = nb;
    }
    const uint64_t cap_bmp_words = static_cast<uint64_t>(caps.bmp) * 1024u;
    const OutLayout L = plan_out(bound, 0, cap_bmp_words, caps.arr, caps.run_u16);
    CR_RET(alloc_out(out, L, bound, 0, cap_bmp_words, caps.arr, caps.run_u16, s));
    HostSlotGuard hs;
    CR_RET(hs.acquire());
    {
        SetOpPlan P;
        if (only_bb && a->key_index && b->key_index) {
            CR_RET(plan_bitmap_keyed(a, b, op, bound, caps, s, P));
        } else {
            CR_RET(plan_set_operation(A, B, op, bound, caps, s, P));
        }
        CR_RET(exec_set_operation(A, B, op, bound, std::min(caps.bmp, bound), std::min(caps.small, bound), only_bb, P,
                                  out, hs.dev<SetOpHost>(), s));
        CR_RET(sync_stream(s));
    }
    const volatile SetOpHost* h = hs.host<SetOpHost>();
    uint32_t c[C_N];
    for (int k = 0; k < C_N; ++k) c[k] = h->c[k];
    const uint32_t n_out = h->n_out, overflow = h->overflow;
    if (overflow || c[C_ITEM] == 0) {
        free_async(out, s);
        reset(out);
        out->universe_size = std::max(a->universe_size, b->universe_size);
        out->negated = neg;
        if (c[C_ITEM] == 0 && !overflow) return CR_OK;
        return set_operation_exact(a, b, A, B, op, bound, s, out);  // counts that do not describe the inputs
    }
    set_counts(out, c);
    out->n_containers = n_out;
    // total_cardinality, key_index and max_key stay 0/null (src/set_ops.cu:1162-1175).
    return CR_OK;
}

// ---- fused multi_and over all-bitmap inputs ---------------------------------
constexpr int MAX_FUSED = 32;

struct FusedIn {
    const uint16_t* keys;
    const uint64_t* bmp;
    const uint16_t* kidx;
    uint32_t n;
    uint32_t kidx_len;  // max_key + 1 when key_index is present, else 0
};

struct FusedArgs {
    FusedIn in[MAX_FUSED];
    uint32_t count;
    uint32_t neg_mask;
};

// Common keys: AND of the key-presence sets of the non-negated inputs, or the
// universe mask [0, mkp1) when every input is negated (src/set_ops.cu:1239-1264).
// Two passes over the 65536-key space in 64 ranges of 1024 keys:
//   mand_presence  (range, input): the input's sorted keys inside the range
//                  become 32 presence words (no global atomics);
//   mand_common    (range): AND over inputs, rank base = popcount of the AND
//                  of all earlier words, one thread per key writes its rank.
constexpr uint32_t KEY_RANGES = 64;

__global__ __launch_bounds__(256) void mand_presence(FusedArgs args, uint32_t* gpres)
{
    __shared__ uint32_t words[32];
    __shared__ uint32_t range[2];
    const uint32_t r = blockIdx.x, k = blockIdx.y, t = threadIdx.x;
    if ((args.neg_mask >> k) & 1u) return;  // only non-negated inputs restrict the key set
    const uint32_t base = r * 1024u;
    if (t < 32) words[t] = 0;
    if (t < 128) {  // waves 0 and 1 find the input's index range for [base, base + 1024)
        const uint32_t v = wave_lower_bound_u16(args.in[k].keys, args.in[k].keys ? args.in[k].n : 0u,
                                                base + (t >= 64 ? 1024u : 0u));
        if ((t & 63u) == 0) range[t >> 6] = v;
    }
    __syncthreads();
    for (uint32_t j = range[0] + t; j < range[1]; j += 256u) {
        const uint32_t off = args.in[k].keys[j] - base;
        if (off < 1024u) atomicOr(&words[off >> 5], 1u << (off & 31u));
    }
    __syncthreads();
    if (t < 32) gpres[k * 2048u + r * 32u + t] = words[t];
}

__device__ __forceinline__ uint32_t common_word(const FusedArgs& args, const uint32_t* gpres, bool any_plain,
                                                uint32_t mkp1, uint32_t j)
{
    if (!any_plain) {
        const uint32_t lo = j * 32u;
        return lo >= mkp1 ? 0u : (lo + 32u <= mkp1 ? ~0u : ((1u << (mkp1 - lo)) - 1u));
    }
    uint32_t acc = ~0u;
    for (uint32_t k = 0; k < args.count; ++k)
        if (!((args.neg_mask >> k) & 1u)) acc &= gpres[k * 2048u + j];
    return acc;
}

__global__ __launch_bounds__(1024) void mand_common(FusedArgs args, const uint32_t* gpres, uint32_t mkp1,
                                                    uint16_t* common, uint32_t* n_common)
{
    __shared__ uint32_t lds[16];
    const uint32_t w = blockIdx.x, t = threadIdx.x;
    const uint32_t all = args.count >= 32 ? ~0u : ((1u << args.count) - 1u);
    const bool any_plain = (args.neg_mask & all) != all;
    uint32_t before = 0;
    for (uint32_t j = t; j < w * 32u; j += 1024u) before += __popc(common_word(args, gpres, any_plain, mkp1, j));
    before = block_sum<1024>(before, lds);
    const uint32_t key = w * 1024u + t;
    const bool present = (common_word(args, gpres, any_plain, mkp1, key >> 5) >> (key & 31u)) & 1u;
    uint32_t here;
    const uint32_t rank = before + block_excl_scan<1024>(present ? 1u : 0u, lds, here);
    if (present) common[rank] = static_cast<uint16_t>(key);
    if (t == 0 && w == KEY_RANGES - 1) *n_common = before + here;
}

__device__ __forceinline__ int32_t fused_lookup(const FusedIn& in, uint32_t key)
{
    if (in.n == 0 || in.keys == nullptr) return -1;
    if (in.kidx && key < in.kidx_len) {  // src/set_ops.cu:1369-1373
        const uint32_t v = in.kidx[key];
        return v == 0xFFFFu ? -1 : static_cast<int32_t>(v);
    }
    uint32_t lo = 0, hi = in.n;  // binary search fallback (:1375-1383)
    while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        const uint32_t k = in.keys[mid];
        if (k < key)
            lo = mid + 1;
        else if (k > key)
            hi = mid;
        else
            return static_cast<int32_t>(mid);
    }
    return -1;
}

__global__ __launch_bounds__(EXEC_NT) void mand_and(FusedArgs args, const uint16_t* common, const uint32_t* n_common_p,
                                                    uint32_t cap, uint64_t* out_bmp, uint16_t* keys, uint8_t* types,
                                                    uint32_t* offsets, uint16_t* cards, uint16_t* key_index,
                                                    uint32_t kidx_len, uint32_t* total)
{
    // One wavefront per common key: lane k resolves input k's container, the wave
    // then streams every input's 8 KiB (8 x 16-byte loads per lane per input)
    // into a register accumulator.  The total cardinality is summed per wave and
    // added once per workgroup.
    __shared__ uint32_t wave_total[EXEC_NT / 64];
    const uint32_t n_common = min(*n_common_p, cap);  // cap: the containers the output was allocated for
    const uint32_t lane = __lane_id();
    const uint32_t n_waves = gridDim.x * (EXEC_NT / 64);
    uint32_t my_total = 0;
    for (uint32_t c = (blockIdx.x * EXEC_NT + threadIdx.x) >> 6; c < n_common; c += n_waves) {
        const uint32_t key = common[c];
        // The container is addressed by its index (bitmap_data + idx * 1024,
        // src/set_ops.cu:1390), not by its offset; an absent key reads as the
        // all-zeros sentinel, which a negated input turns into all-ones.
        const int32_t my_idx = lane < args.count ? fused_lookup(args.in[lane], key) : -1;
        uint4 acc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = make_uint4(~0u, ~0u, ~0u, ~0u);
        // Input k + 1's eight 16-byte loads are issued before input k is ANDed
        // in, so a wave keeps two inputs' reads in flight.
        auto src_of = [&](uint32_t k, int32_t& idx) -> const uint64_t* {
            idx = __shfl(my_idx, static_cast<int>(k), 64);
            return idx < 0 ? nullptr : args.in[k].bmp + static_cast<uint64_t>(idx) * 1024u;
        };
        auto load8 = [&](const uint64_t* p, uint4 (&x)[8]) {
            if (!p) return;
            if ((reinterpret_cast<uintptr_t>(p) & 15u) == 0) {
                const uint4* p4 = reinterpret_cast<const uint4*>(p);
#pragma unroll
                for (int j = 0; j < 8; ++j) x[j] = ld_stream(p4 + lane + 64 * j);
            } else {
                const uint32_t* p32 = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint32_t b = 4 * (lane + 64 * j);
                    x[j] = make_uint4(p32[b], p32[b + 1], p32[b + 2], p32[b + 3]);
                }
            }
        };
        uint4 cur[8], nxt[8];
        int32_t idx_cur = -1, idx_nxt = -1;
        const uint64_t* p_cur = args.count ? src_of(0, idx_cur) : nullptr;
        load8(p_cur, cur);
        for (uint32_t k = 0; k < args.count; ++k) {
            const uint64_t* p_nxt = k + 1 < args.count ? src_of(k + 1, idx_nxt) : nullptr;
            load8(p_nxt, nxt);
            const bool neg = (args.neg_mask >> k) & 1u;
            if (idx_cur < 0) {
                if (!neg) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) acc[j] = make_uint4(0, 0, 0, 0);
                }
            } else {
                const uint32_t m = neg ? ~0u : 0u;
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    acc[j] = make_uint4(acc[j].x & (cur[j].x ^ m), acc[j].y & (cur[j].y ^ m), acc[j].z & (cur[j].z ^ m),
                                        acc[j].w & (cur[j].w ^ m));
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) cur[j] = nxt[j];
            idx_cur = idx_nxt;
        }
        uint4* dst = reinterpret_cast<uint4*>(out_bmp + static_cast<uint64_t>(c) * 1024u);
        uint32_t pc = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            st_stream(dst + lane + 64 * j, acc[j]);
            pc += __popc(acc[j].x) + __popc(acc[j].y) + __popc(acc[j].z) + __popc(acc[j].w);
        }
        pc = wave_sum(pc);
        my_total += pc;
        if (lane == 0) {
            cards[c] = static_cast<uint16_t>(pc > 65535u ? 65535u : pc);  // clamp (src/set_ops.cu:1468)
            keys[c] = static_cast<uint16_t>(key);
            types[c] = CR_BITMAP;
            offsets[c] = c * 8192u;
            // The index is sized from the universe; a key beyond it (a bitset upload
            // whose words outrun U) has no slot -- the reference writes out of bounds.
            if (key < kidx_len) key_index[key] = static_cast<uint16_t>(c);
        }
    }
    if (lane == 0) wave_total[threadIdx.x >> 6] = my_total;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t s = 0;
        for (int i = 0; i < EXEC_NT / 64; ++i) s += wave_total[i];
        if (s) atomicAdd(total, s);  // u32 like the reference's counter (src/set_ops.cu:1652-1654)
    }
}

// n_common and the total cardinality, for the host's one read after the sync.
__global__ void mand_finish(const uint32_t* cnt, uint32_t* host)
{
    volatile uint32_t* h = host;
    h[0] = cnt[0];
    h[1] = cnt[1];
}

static int fused_multi_and(const cr_gpu_roaring* in, uint32_t count, hipStream_t s, cr_gpu_roaring* out)
{
    FusedArgs args{};
    args.count = count;
    uint32_t universe = in[0].universe_size;
    for (uint32_t i = 0; i < count; ++i) {
        if (in[i].negated) args.neg_mask |= 1u << i;
        universe = std::max(universe, in[i].universe_size);
        args.in[i].keys = in[i].keys;
        args.in[i].bmp = in[i].bitmap_data;
        args.in[i].kidx = in[i].key_index;
        args.in[i].n = in[i].n_containers;
        args.in[i].kidx_len = in[i].key_index ? in[i].max_key + 1u : 0u;
    }
    uint32_t mkp1 = static_cast<uint32_t>(universe + 65535u) / 65536u;  // u32 arithmetic (:1506)
    if (mkp1 > 65536u) mkp1 = 65536u;
    reset(out);
    out->universe_size = universe;

    Carver c;
    const size_t o_common = c.add(2 * 65536);
    const size_t o_cnt = c.add(2 * sizeof(uint32_t));
    const size_t o_pres = c.add(sizeof(uint32_t) * 2048u * count);
    Scratch sc;
    CR_RET(sc.alloc(c.total, s));
    uint16_t* common = sc.at<uint16_t>(o_common);
    uint32_t* cnt = sc.at<uint32_t>(o_cnt);  // [0] n_common, [1] total cardinality
    uint32_t* gpres = sc.at<uint32_t>(o_pres);
    {
        CR_TIMED("mand_keys", s);
        mand_presence<<<dim3(KEY_RANGES, count), 256, 0, s>>>(args, gpres);
        mand_common<<<KEY_RANGES, 1024, 0, s>>>(args, gpres, mkp1, common, cnt);
    }
    CR_LAUNCH_CHECK();
    CR_RET(fill_u32(cnt + 1, 0u, 1, s));

    // One synchronisation: the output is allocated for the most common keys
    // there can be -- the fewest containers of a non-negated input (the common
    // keys are a subset of each one's keys), or every key of the universe when
    // all inputs are negated -- before they are counted.
    uint32_t cap = 0xFFFFFFFFu;
    for (uint32_t i = 0; i < count; ++i)
        if (!in[i].negated) cap = std::min(cap, in[i].n_containers);
    if (cap == 0xFFFFFFFFu) cap = mkp1;
    const uint32_t max_key = mkp1 == 0 ? 0u : mkp1 - 1u;
    const uint64_t kidx_len = static_cast<uint64_t>(max_key) + 1u;
    HostSlotGuard hs;
    CR_RET(hs.acquire());
    if (cap > 0) {
        const OutLayout L = plan_out(cap, kidx_len, static_cast<uint64_t>(cap) * 1024u, 0, 0);
        CR_RET(alloc_out(out, L, cap, kidx_len, static_cast<uint64_t>(cap) * 1024u, 0, 0, s));
        out->max_key = max_key;
        CR_RET(fill_u16(out->key_index, 0xFFFFu, kidx_len, s));
        CR_TIMED("mand_and", s);
        // One common key per wave (a grid capped at 8 workgroups per CU, two
        // keys a wave, measured 0.69 of peak against 0.71 at k = 3); waves past
        // the common keys exit.
        const unsigned gm = std::max(1u, (cap + 3) / 4);
        mand_and<<<gm, EXEC_NT, 0, s>>>(args, common, cnt, cap, out->bitmap_data, out->keys, out->types,
                                        out->offsets, out->cardinalities, out->key_index,
                                        static_cast<uint32_t>(kidx_len), cnt + 1);
    }
    CR_LAUNCH_CHECK();
    mand_finish<<<1, 1, 0, s>>>(cnt, hs.dev<uint32_t>());
    CR_LAUNCH_CHECK();
    CR_RET(sync_stream(s));
    const volatile uint32_t* h = hs.host<uint32_t>();
    const uint32_t h0 = h[0], total = h[1];
    const uint32_t n_common = std::min(h0, cap);
    if (n_common == 0) {  // src/set_ops.cu:1579-1583
        free_async(out, s);
        reset(out);
        out->universe_size = universe;
        return CR_OK;
    }
    out->n_containers = n_common;
    out->n_bitmap_containers = n_common;
    out->total_cardinality = total;
    return CR_OK;
}

int multi_and_impl(const cr_gpu_roaring* in, uint32_t count, hipStream_t s, cr_gpu_roaring* out)
{
    reset(out);
    if (count == 0) return CR_OK;  // src/set_ops.cu:1718
    if (count == 1) return set_operation_impl(&in[0], &in[0], CR_AND, s, out);
    bool all_bitmap = true;
    for (uint32_t i = 0; i < count; ++i)
        if (in[i].n_array_containers > 0 || in[i].n_run_containers > 0) all_bitmap = false;
    if (all_bitmap && count <= MAX_FUSED) return fused_multi_and(in, count, s, out);
    cr_gpu_roaring acc;
    CR_RET(set_operation_impl(&in[0], &in[1], CR_AND, s, &acc));
    for (uint32_t i = 2; i < count; ++i) {
        cr_gpu_roaring next;
        const int rc = set_operation_impl(&acc, &in[i], CR_AND, s, &next);
        free_async(&acc, s);
        if (rc != CR_OK) return rc;
        acc = next;
    }
    *out = acc;
    return CR_OK;
}

}  // namespace crimpl

using namespace crimpl;

extern "C" int cr_set_operation(const cr_gpu_roaring* a, const cr_gpu_roaring* b, uint32_t op, cr_stream_t stream,
                                cr_gpu_roaring* out)
{
    if (!a || !b || !out || op > CR_XOR) {
        set_error("cr_set_operation: invalid argument");
        return CR_ERR_INVALID;
    }
    reset(out);
    return produced(set_operation_impl(a, b, op, as_stream(stream), out), out, as_stream(stream));
}

extern "C" int cr_multi_and(const cr_gpu_roaring* bitmaps, uint32_t count, cr_stream_t stream, cr_gpu_roaring* out)
{
    if (!out || (count > 0 && !bitmaps)) {
        set_error("cr_multi_and: invalid argument");
        return CR_ERR_INVALID;
    }
    reset(out);
    return produced(multi_and_impl(bitmaps, count, as_stream(stream), out), out, as_stream(stream));
}

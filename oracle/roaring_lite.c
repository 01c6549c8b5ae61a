/*
 * roaring_lite.c -- a small host Roaring bitmap (TEST INFRASTRUCTURE ONLY).
 *
 * CRoaring (the reference's CPU oracle and CPU baseline, third_party/CRoaring)
 * is not present in the reference checkout (.gitmodules:1-3 pins no commit and
 * the directory is empty), so this file restates the public Roaring format
 * rules the reference relies on:
 *   - containers keyed by the high 16 bits, sorted by key;
 *   - array container iff cardinality <= 4096, else bitset (1024 x u64);
 *   - run_optimize: a container becomes a run container iff its serialized
 *     run size (2 + 4*n_runs bytes) is smaller than its current serialized size
 *     (array: 2 + 2*card bytes, bitset: 8192 bytes);
 *   - runs are (start, length) pairs covering [start, start+length].
 * Set-operation results are typed array/bitset by cardinality only; CRoaring
 * may keep run containers in some results -- its exact type choices are not
 * pinned by any reference test (they compare decoded bitsets only).
 *
 * Pinning: tests/test_oracle_lite.py checks every operation against a
 * flat-bitset brute force on random inputs (uniform, clustered, full and empty
 * containers, the 65535/65536 boundary) and the run_optimize decision against
 * the serialized-size rule computed independently in numpy.  The portable
 * format writer and reader are pinned by byte strings assembled in the test
 * from the format specification (cookies, run flags, the offset-header rule,
 * card-1, each payload kind) and by round trips.
 *
 * The same code is the CPU baseline ("port") that bench.py times: merge /
 * galloping array intersection, word-wise bitset ops with popcount.
 */
#include "oracle.h"

#include <stdlib.h>
#include <string.h>

#define ARRAY_MAX 4096

static int popc64(uint64_t x) { return __builtin_popcountll(x); }

rl_bitmap* rl_create(void) { return (rl_bitmap*)calloc(1, sizeof(rl_bitmap)); }

static void rl_reserve(rl_bitmap* b, uint32_t need)
{
    if (need <= b->cap) return;
    uint32_t cap = b->cap ? b->cap * 2 : 16;
    while (cap < need) cap *= 2;
    b->keys = (uint16_t*)realloc(b->keys, cap * sizeof(uint16_t));
    b->tc = (uint8_t*)realloc(b->tc, cap);
    b->card = (int32_t*)realloc(b->card, cap * sizeof(int32_t));
    b->data = (void**)realloc(b->data, cap * sizeof(void*));
    b->cap = cap;
}

static void rl_push(rl_bitmap* b, uint16_t key, uint8_t tc, int32_t card, void* data)
{
    rl_reserve(b, b->n + 1);
    b->keys[b->n] = key;
    b->tc[b->n] = tc;
    b->card[b->n] = card;
    b->data[b->n] = data;
    b->n++;
}

void rl_destroy(rl_bitmap* b)
{
    if (!b) return;
    for (uint32_t i = 0; i < b->n; ++i) free(b->data[i]);
    free(b->keys);
    free(b->tc);
    free(b->card);
    free(b->data);
    free(b);
}

/* Make a container of the right type from a 1024-word bitset (takes ownership
 * of `bits` or frees it). */
static void push_from_bits(rl_bitmap* r, uint16_t key, uint64_t* bits, int32_t card)
{
    if (card == 0) {
        free(bits);
        return;
    }
    if (card <= ARRAY_MAX) {
        uint16_t* a = (uint16_t*)malloc((size_t)card * 2u);
        int32_t k = 0;
        for (uint32_t w = 0; w < 1024u; ++w) {
            uint64_t x = bits[w];
            while (x) {
                a[k++] = (uint16_t)(w * 64u + (uint32_t)__builtin_ctzll(x));
                x &= x - 1;
            }
        }
        free(bits);
        rl_push(r, key, ORC_TC_ARRAY, card, a);
    } else {
        rl_push(r, key, ORC_TC_BITSET, card, bits);
    }
}

static void push_from_array(rl_bitmap* r, uint16_t key, uint16_t* vals, int32_t card)
{
    if (card == 0) {
        free(vals);
        return;
    }
    if (card <= ARRAY_MAX) {
        rl_push(r, key, ORC_TC_ARRAY, card, vals);
        return;
    }
    uint64_t* bits = (uint64_t*)calloc(1024, 8);
    for (int32_t i = 0; i < card; ++i) bits[vals[i] >> 6] |= 1ull << (vals[i] & 63u);
    free(vals);
    rl_push(r, key, ORC_TC_BITSET, card, bits);
}

rl_bitmap* rl_from_sorted_ids(const uint32_t* ids, uint64_t n)
{
    rl_bitmap* r = rl_create();
    uint64_t s = 0;
    while (s < n) {
        uint32_t key = ids[s] >> 16;
        uint64_t e = s;
        while (e < n && (ids[e] >> 16) == key) ++e;
        int32_t card = (int32_t)(e - s);
        if (card <= ARRAY_MAX) {
            uint16_t* a = (uint16_t*)malloc((size_t)card * 2u);
            for (uint64_t i = s; i < e; ++i) a[i - s] = (uint16_t)ids[i];
            rl_push(r, (uint16_t)key, ORC_TC_ARRAY, card, a);
        } else {
            uint64_t* bits = (uint64_t*)calloc(1024, 8);
            for (uint64_t i = s; i < e; ++i) {
                uint32_t v = ids[i] & 0xFFFFu;
                bits[v >> 6] |= 1ull << (v & 63u);
            }
            rl_push(r, (uint16_t)key, ORC_TC_BITSET, card, bits);
        }
        s = e;
    }
    return r;
}

/* A flat bitset of n_words u64 (bit i = id i) as containers, typed by
 * cardinality (array <= 4096, else bitset). */
rl_bitmap* rl_from_words(const uint64_t* words, uint64_t n_words)
{
    rl_bitmap* r = rl_create();
    for (uint64_t w0 = 0; w0 < n_words; w0 += 1024u) {
        uint64_t* bits = (uint64_t*)calloc(1024, 8);
        const uint64_t nw = n_words - w0 < 1024u ? n_words - w0 : 1024u;
        memcpy(bits, words + w0, (size_t)nw * 8u);
        int32_t card = 0;
        for (uint32_t w = 0; w < 1024u; ++w) card += popc64(bits[w]);
        push_from_bits(r, (uint16_t)(w0 >> 10), bits, card);
    }
    return r;
}

static int cmp_u32(const void* a, const void* b)
{
    uint32_t x = *(const uint32_t*)a, y = *(const uint32_t*)b;
    return (x > y) - (x < y);
}

rl_bitmap* rl_from_ids(const uint32_t* ids, uint64_t n)
{
    uint32_t* v = (uint32_t*)malloc((size_t)(n ? n : 1) * 4u);
    if (n) { /* an empty input may come with a null pointer */
        memcpy(v, ids, (size_t)n * 4u);
        qsort(v, n, 4, cmp_u32);
    }
    uint64_t w = 0;
    for (uint64_t i = 0; i < n; ++i)
        if (w == 0 || v[i] != v[w - 1]) v[w++] = v[i];
    rl_bitmap* r = rl_from_sorted_ids(v, w);
    free(v);
    return r;
}

static void* dup_data(uint8_t tc, int32_t card, const void* d)
{
    size_t sz = tc == ORC_TC_BITSET ? 8192u : (tc == ORC_TC_ARRAY ? (size_t)card * 2u : (size_t)card * 4u);
    void* p = malloc(sz ? sz : 1);
    memcpy(p, d, sz);
    return p;
}

rl_bitmap* rl_copy(const rl_bitmap* b)
{
    rl_bitmap* r = rl_create();
    for (uint32_t i = 0; i < b->n; ++i) rl_push(r, b->keys[i], b->tc[i], b->card[i], dup_data(b->tc[i], b->card[i], b->data[i]));
    return r;
}

/* Expand any container to a fresh 1024-word bitset. */
static uint64_t* to_bits(uint8_t tc, int32_t card, const void* d)
{
    uint64_t* bits = (uint64_t*)calloc(1024, 8);
    if (tc == ORC_TC_BITSET) {
        memcpy(bits, d, 8192);
    } else if (tc == ORC_TC_ARRAY) {
        const uint16_t* a = (const uint16_t*)d;
        for (int32_t i = 0; i < card; ++i) bits[a[i] >> 6] |= 1ull << (a[i] & 63u);
    } else {
        const uint16_t* runs = (const uint16_t*)d;
        for (int32_t k = 0; k < card; ++k) {
            uint32_t s = runs[2 * k], e = s + runs[2 * k + 1];
            if (e > 0xFFFFu) e = 0xFFFFu;
            uint32_t ws = s >> 6, we = e >> 6;
            for (uint32_t w = ws; w <= we; ++w) {
                uint64_t m = ~0ull;
                if (w == ws) m &= ~0ull << (s & 63u);
                if (w == we) m &= ~0ull >> (63u - (e & 63u));
                bits[w] |= m;
            }
        }
    }
    return bits;
}

static int32_t bits_card(const uint64_t* bits)
{
    int32_t c = 0;
    for (uint32_t w = 0; w < 1024u; ++w) c += popc64(bits[w]);
    return c;
}

static int32_t runs_in_bits(const uint64_t* bits)
{
    /* number of maximal runs = number of 0->1 transitions */
    int32_t n = 0;
    uint64_t prev_top = 0;
    for (uint32_t w = 0; w < 1024u; ++w) {
        uint64_t x = bits[w];
        uint64_t starts = x & ~((x << 1) | prev_top);
        n += popc64(starts);
        prev_top = x >> 63;
    }
    return n;
}

static uint16_t* bits_to_runs(const uint64_t* bits, int32_t n_runs)
{
    uint16_t* runs = (uint16_t*)malloc((size_t)(n_runs ? n_runs : 1) * 4u);
    int32_t k = 0;
    int32_t v = 0;
    while (v < 65536 && k < n_runs) {
        while (v < 65536 && !((bits[v >> 6] >> (v & 63)) & 1u)) ++v;
        if (v >= 65536) break;
        int32_t s = v;
        while (v < 65536 && ((bits[v >> 6] >> (v & 63)) & 1u)) ++v;
        runs[2 * k] = (uint16_t)s;
        runs[2 * k + 1] = (uint16_t)(v - 1 - s);
        ++k;
    }
    return runs;
}

void rl_run_optimize(rl_bitmap* b)
{
    for (uint32_t i = 0; i < b->n; ++i) {
        if (b->tc[i] == ORC_TC_RUN) continue;
        uint64_t* bits = to_bits(b->tc[i], b->card[i], b->data[i]);
        int32_t nr = runs_in_bits(bits);
        int32_t run_size = 2 + 4 * nr;
        int32_t cur_size = b->tc[i] == ORC_TC_ARRAY ? 2 + 2 * b->card[i] : 8192;
        if (run_size < cur_size) {
            uint16_t* runs = bits_to_runs(bits, nr);
            free(b->data[i]);
            b->data[i] = runs;
            b->tc[i] = ORC_TC_RUN;
            b->card[i] = nr;
        }
        free(bits);
    }
}

/* ---- set operations --------------------------------------------------- */

static int32_t gallop(const uint16_t* a, int32_t n, int32_t pos, uint16_t v)
{
    /* smallest index >= pos with a[idx] >= v */
    int32_t step = 1, lo = pos, hi = pos;
    while (hi < n && a[hi] < v) {
        lo = hi + 1;
        hi += step;
        step <<= 1;
    }
    if (hi > n) hi = n;
    while (lo < hi) {
        int32_t mid = (lo + hi) >> 1;
        if (a[mid] < v)
            lo = mid + 1;
        else
            hi = mid;
    }
    return lo;
}

static int32_t array_and(const uint16_t* a, int32_t na, const uint16_t* b, int32_t nb, uint16_t* out)
{
    if (na > nb) {
        const uint16_t* t = a;
        a = b;
        b = t;
        int32_t tn = na;
        na = nb;
        nb = tn;
    }
    int32_t k = 0;
    if ((int64_t)na * 32 < nb) { /* galloping for skewed sizes */
        int32_t pos = 0;
        for (int32_t i = 0; i < na && pos < nb; ++i) {
            pos = gallop(b, nb, pos, a[i]);
            if (pos < nb && b[pos] == a[i]) out[k++] = a[i];
        }
        return k;
    }
    int32_t i = 0, j = 0;
    while (i < na && j < nb) {
        if (a[i] < b[j])
            ++i;
        else if (a[i] > b[j])
            ++j;
        else {
            out[k++] = a[i];
            ++i;
            ++j;
        }
    }
    return k;
}

static int32_t array_merge(const uint16_t* a, int32_t na, const uint16_t* b, int32_t nb, int op,
                           uint16_t* out)
{
    int32_t i = 0, j = 0, k = 0;
    while (i < na || j < nb) {
        if (j >= nb || (i < na && a[i] < b[j])) {
            if (op != ORC_AND) out[k++] = a[i];
            ++i;
        } else if (i >= na || a[i] > b[j]) {
            if (op == ORC_OR || op == ORC_XOR) out[k++] = b[j];
            ++j;
        } else {
            if (op == ORC_OR) out[k++] = a[i];
            ++i;
            ++j;
        }
    }
    return k;
}

static void container_op(rl_bitmap* r, uint16_t key, uint8_t ta, int32_t ca, const void* da,
                         uint8_t tb, int32_t cb, const void* db, int op)
{
    if (ta == ORC_TC_ARRAY && tb == ORC_TC_ARRAY) {
        if (op == ORC_AND) {
            uint16_t* out = (uint16_t*)malloc((size_t)((ca < cb ? ca : cb) + 1) * 2u);
            int32_t k = array_and((const uint16_t*)da, ca, (const uint16_t*)db, cb, out);
            push_from_array(r, key, out, k);
        } else {
            uint16_t* out = (uint16_t*)malloc((size_t)(ca + cb + 1) * 2u);
            int32_t k = array_merge((const uint16_t*)da, ca, (const uint16_t*)db, cb, op, out);
            push_from_array(r, key, out, k);
        }
        return;
    }
    if (op == ORC_AND && (ta == ORC_TC_ARRAY || tb == ORC_TC_ARRAY) &&
        (ta == ORC_TC_BITSET || tb == ORC_TC_BITSET)) {
        const uint16_t* arr = (const uint16_t*)(ta == ORC_TC_ARRAY ? da : db);
        int32_t n = ta == ORC_TC_ARRAY ? ca : cb;
        const uint64_t* bits = (const uint64_t*)(ta == ORC_TC_BITSET ? da : db);
        uint16_t* out = (uint16_t*)malloc((size_t)(n + 1) * 2u);
        int32_t k = 0;
        for (int32_t i = 0; i < n; ++i)
            if ((bits[arr[i] >> 6] >> (arr[i] & 63u)) & 1u) out[k++] = arr[i];
        push_from_array(r, key, out, k);
        return;
    }
    uint64_t* x = to_bits(ta, ca, da);
    uint64_t* y = (tb == ORC_TC_BITSET) ? NULL : to_bits(tb, cb, db);
    const uint64_t* yy = y ? y : (const uint64_t*)db;
    int32_t card = 0;
    switch (op) {
    case ORC_AND:
        for (uint32_t w = 0; w < 1024u; ++w) card += popc64(x[w] &= yy[w]);
        break;
    case ORC_OR:
        for (uint32_t w = 0; w < 1024u; ++w) card += popc64(x[w] |= yy[w]);
        break;
    case ORC_ANDNOT:
        for (uint32_t w = 0; w < 1024u; ++w) card += popc64(x[w] &= ~yy[w]);
        break;
    default:
        for (uint32_t w = 0; w < 1024u; ++w) card += popc64(x[w] ^= yy[w]);
        break;
    }
    free(y);
    push_from_bits(r, key, x, card);
}

static void push_copy(rl_bitmap* r, const rl_bitmap* s, uint32_t i)
{
    rl_push(r, s->keys[i], s->tc[i], s->card[i], dup_data(s->tc[i], s->card[i], s->data[i]));
}

rl_bitmap* rl_op(const rl_bitmap* a, const rl_bitmap* b, int op)
{
    rl_bitmap* r = rl_create();
    uint32_t i = 0, j = 0;
    while (i < a->n || j < b->n) {
        if (j >= b->n || (i < a->n && a->keys[i] < b->keys[j])) {
            if (op != ORC_AND) push_copy(r, a, i);
            ++i;
        } else if (i >= a->n || a->keys[i] > b->keys[j]) {
            if (op == ORC_OR || op == ORC_XOR) push_copy(r, b, j);
            ++j;
        } else {
            container_op(r, a->keys[i], a->tc[i], a->card[i], a->data[i], b->tc[j], b->card[j],
                         b->data[j], op);
            ++i;
            ++j;
        }
    }
    return r;
}

/* The containers of keys [key_lo, key_hi), copied (a shard by key range). */
rl_bitmap* rl_slice(const rl_bitmap* b, uint32_t key_lo, uint32_t key_hi)
{
    rl_bitmap* r = rl_create();
    for (uint32_t i = 0; i < b->n; ++i)
        if (b->keys[i] >= key_lo && b->keys[i] < key_hi) push_copy(r, b, i);
    return r;
}

/* Complement of [lo, hi) (roaring_bitmap_flip).  Containers outside the range
 * are copied; inside, bits are inverted and the result retyped by cardinality. */
rl_bitmap* rl_flip(const rl_bitmap* b, uint64_t lo, uint64_t hi)
{
    rl_bitmap* r = rl_create();
    if (hi <= lo) {
        rl_bitmap* c = rl_copy(b);
        rl_destroy(r);
        return c;
    }
    uint32_t k_lo = (uint32_t)(lo >> 16), k_hi = (uint32_t)((hi - 1) >> 16);
    uint32_t i = 0;
    for (uint32_t key = 0; key <= 65535u; ++key) {
        int has = i < b->n && b->keys[i] == key;
        if (key < k_lo || key > k_hi) {
            if (has) push_copy(r, b, i);
        } else {
            uint64_t* bits = has ? to_bits(b->tc[i], b->card[i], b->data[i]) : (uint64_t*)calloc(1024, 8);
            uint64_t base = (uint64_t)key << 16;
            uint64_t s = lo > base ? lo - base : 0, e = hi - base; /* flip [s, e) */
            if (e > 65536u) e = 65536u;
            for (uint64_t w = s >> 6; w < ((e + 63u) >> 6); ++w) {
                uint64_t m = ~0ull;
                if (w == (s >> 6)) m &= ~0ull << (s & 63u);
                if (w == ((e - 1u) >> 6) && (e & 63u)) m &= (1ull << (e & 63u)) - 1ull;
                bits[w] ^= m;
            }
            push_from_bits(r, (uint16_t)key, bits, bits_card(bits));
        }
        if (has) ++i;
        if (key == 65535u) break;
    }
    return r;
}

static int container_contains(uint8_t tc, int32_t card, const void* d, uint16_t low)
{
    if (tc == ORC_TC_BITSET) return (int)((((const uint64_t*)d)[low >> 6] >> (low & 63u)) & 1u);
    if (tc == ORC_TC_ARRAY) {
        const uint16_t* a = (const uint16_t*)d;
        int32_t lo = 0, hi = card - 1;
        while (lo <= hi) {
            int32_t mid = (lo + hi) >> 1;
            if (a[mid] == low) return 1;
            if (a[mid] < low)
                lo = mid + 1;
            else
                hi = mid - 1;
        }
        return 0;
    }
    const uint16_t* runs = (const uint16_t*)d;
    int32_t lo = 0, hi = card - 1;
    while (lo <= hi) {
        int32_t mid = (lo + hi) >> 1;
        uint32_t s = runs[2 * mid], l = runs[2 * mid + 1];
        if (low < s)
            hi = mid - 1;
        else if (low > s + l)
            lo = mid + 1;
        else
            return 1;
    }
    return 0;
}

int rl_contains(const rl_bitmap* b, uint32_t id)
{
    uint16_t key = (uint16_t)(id >> 16);
    int32_t lo = 0, hi = (int32_t)b->n - 1;
    while (lo <= hi) {
        int32_t mid = (lo + hi) >> 1;
        if (b->keys[mid] == key) return container_contains(b->tc[mid], b->card[mid], b->data[mid], (uint16_t)id);
        if (b->keys[mid] < key)
            lo = mid + 1;
        else
            hi = mid - 1;
    }
    return 0;
}

void rl_contains_many(const rl_bitmap* b, const uint32_t* ids, uint64_t n, uint32_t* out)
{
    for (uint64_t i = 0; i < n; ++i) out[i] = (uint32_t)rl_contains(b, ids[i]);
}

static uint64_t container_card(uint8_t tc, int32_t card, const void* d)
{
    if (tc != ORC_TC_RUN) return (uint64_t)card;
    const uint16_t* runs = (const uint16_t*)d;
    uint64_t t = 0;
    for (int32_t k = 0; k < card; ++k) t += (uint64_t)runs[2 * k + 1] + 1u;
    return t;
}

uint64_t rl_cardinality(const rl_bitmap* b)
{
    uint64_t t = 0;
    for (uint32_t i = 0; i < b->n; ++i) t += container_card(b->tc[i], b->card[i], b->data[i]);
    return t;
}

uint64_t rl_to_ids(const rl_bitmap* b, uint32_t* out)
{
    uint64_t k = 0;
    for (uint32_t i = 0; i < b->n; ++i) {
        uint32_t base = (uint32_t)b->keys[i] << 16;
        if (!out) {
            k += container_card(b->tc[i], b->card[i], b->data[i]);
            continue;
        }
        if (b->tc[i] == ORC_TC_ARRAY) {
            const uint16_t* a = (const uint16_t*)b->data[i];
            for (int32_t j = 0; j < b->card[i]; ++j) out[k++] = base | a[j];
        } else {
            uint64_t* bits = to_bits(b->tc[i], b->card[i], b->data[i]);
            for (uint32_t w = 0; w < 1024u; ++w) {
                uint64_t x = bits[w];
                while (x) {
                    out[k++] = base | (w * 64u + (uint32_t)__builtin_ctzll(x));
                    x &= x - 1;
                }
            }
            free(bits);
        }
    }
    return k;
}

uint32_t rl_n_containers(const rl_bitmap* b) { return b->n; }

void rl_container_info(const rl_bitmap* b, uint32_t i, uint16_t* key, uint8_t* tc, int32_t* card,
                       const void** data)
{
    *key = b->keys[i];
    *tc = b->tc[i];
    *card = b->card[i];
    *data = b->data[i];
}

void rl_to_containers(const rl_bitmap* b, orc_container* out)
{
    for (uint32_t i = 0; i < b->n; ++i) {
        out[i].key = b->keys[i];
        out[i].typecode = b->tc[i];
        out[i].card = b->card[i];
        out[i].data = b->data[i];
    }
}

void rl_count_types(const rl_bitmap* b, uint32_t* n_bitset, uint32_t* n_array, uint32_t* n_run)
{
    *n_bitset = *n_array = *n_run = 0;
    for (uint32_t i = 0; i < b->n; ++i) {
        if (b->tc[i] == ORC_TC_BITSET)
            ++*n_bitset;
        else if (b->tc[i] == ORC_TC_ARRAY)
            ++*n_array;
        else
            ++*n_run;
    }
}

/* ---- portable serialization ------------------------------------------------
 * The Roaring portable format (RoaringFormatSpec, the layout CRoaring's
 * roaring_bitmap_portable_serialize writes), all fields little-endian:
 *   cookie   no run container: u32 12346, u32 size;
 *            otherwise: u16 12347, u16 size-1, then ceil(size/8) bytes whose
 *            bit i (LSB first) marks container i as a run container;
 *   header   size x (u16 key, u16 cardinality-1);
 *   offsets  size x u32 byte offsets from the first cookie byte to each payload,
 *            present iff there is no run container or size >= 4;
 *   payloads in container order: run = u16 n_runs + n_runs x (u16 start,
 *            u16 length-1); otherwise cardinality <= 4096: cardinality x u16
 *            sorted values, else the 1024 x u64 bitset.
 * A reader infers the kind from the run bit, then from the cardinality, and
 * reads the payloads in sequence (offsets are not consulted). */
#define PORTABLE_COOKIE_NO_RUN 12346u
#define PORTABLE_COOKIE 12347u
#define PORTABLE_NO_OFFSET_THRESHOLD 4u

static uint32_t rl_true_card(const rl_bitmap* b, uint32_t i)
{
    if (b->tc[i] != ORC_TC_RUN) return (uint32_t)b->card[i];
    const uint16_t* r = (const uint16_t*)b->data[i];
    uint32_t t = 0;
    for (int32_t k = 0; k < b->card[i]; ++k) t += (uint32_t)r[2 * k + 1] + 1u;
    return t;
}

static int rl_has_run(const rl_bitmap* b)
{
    for (uint32_t i = 0; i < b->n; ++i)
        if (b->tc[i] == ORC_TC_RUN) return 1;
    return 0;
}

static uint64_t portable_header_bytes(uint32_t n, int has_run)
{
    uint64_t h = has_run ? 4u + (n + 7u) / 8u : 8u;
    h += 4ull * n;
    if (!has_run || n >= PORTABLE_NO_OFFSET_THRESHOLD) h += 4ull * n;
    return h;
}

static uint64_t portable_payload_bytes(const rl_bitmap* b, uint32_t i)
{
    if (b->tc[i] == ORC_TC_RUN) return 2u + 4ull * (uint32_t)b->card[i];
    const uint32_t card = rl_true_card(b, i);
    return card <= ARRAY_MAX ? 2ull * card : 8192u;
}

uint64_t rl_portable_size(const rl_bitmap* b)
{
    uint64_t t = portable_header_bytes(b->n, rl_has_run(b));
    for (uint32_t i = 0; i < b->n; ++i) t += portable_payload_bytes(b, i);
    return t;
}

static void put16(uint8_t* p, uint32_t v)
{
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
}
static void put32(uint8_t* p, uint32_t v)
{
    put16(p, v & 0xFFFFu);
    put16(p + 2, v >> 16);
}
static uint32_t get16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }
static uint32_t get32(const uint8_t* p) { return get16(p) | (get16(p + 2) << 16); }

uint64_t rl_portable_serialize(const rl_bitmap* b, uint8_t* out)
{
    const uint32_t n = b->n;
    const int has_run = rl_has_run(b);
    uint8_t* p = out;
    if (has_run) {
        put16(p, PORTABLE_COOKIE);
        put16(p + 2, n - 1u);
        p += 4;
        memset(p, 0, (n + 7u) / 8u);
        for (uint32_t i = 0; i < n; ++i)
            if (b->tc[i] == ORC_TC_RUN) p[i / 8u] |= (uint8_t)(1u << (i % 8u));
        p += (n + 7u) / 8u;
    } else {
        put32(p, PORTABLE_COOKIE_NO_RUN);
        put32(p + 4, n);
        p += 8;
    }
    for (uint32_t i = 0; i < n; ++i) {
        put16(p, b->keys[i]);
        put16(p + 2, rl_true_card(b, i) - 1u);
        p += 4;
    }
    uint64_t off = portable_header_bytes(n, has_run);
    if (!has_run || n >= PORTABLE_NO_OFFSET_THRESHOLD) {
        for (uint32_t i = 0; i < n; ++i) {
            put32(p, (uint32_t)off);
            p += 4;
            off += portable_payload_bytes(b, i);
        }
    }
    for (uint32_t i = 0; i < n; ++i) {
        if (b->tc[i] == ORC_TC_RUN) {
            const uint16_t* r = (const uint16_t*)b->data[i];
            put16(p, (uint32_t)b->card[i]);
            p += 2;
            for (int32_t k = 0; k < 2 * b->card[i]; ++k, p += 2) put16(p, r[k]);
            continue;
        }
        const uint32_t card = rl_true_card(b, i);
        uint64_t* bits = to_bits(b->tc[i], b->card[i], b->data[i]);
        if (card <= ARRAY_MAX) {
            for (uint32_t w = 0; w < 1024u; ++w)
                for (uint64_t x = bits[w]; x; x &= x - 1, p += 2) put16(p, w * 64u + (uint32_t)__builtin_ctzll(x));
        } else {
            for (uint32_t w = 0; w < 1024u; ++w, p += 8) {
                put32(p, (uint32_t)bits[w]);
                put32(p + 4, (uint32_t)(bits[w] >> 32));
            }
        }
        free(bits);
    }
    return (uint64_t)(p - out);
}

/* NULL when `buf` is not a well-formed portable bitmap of at most `len` bytes
 * (truncated, bad cookie, keys not strictly increasing, a run past 0xFFFF). */
rl_bitmap* rl_portable_deserialize(const uint8_t* buf, uint64_t len, uint64_t* consumed)
{
    if (len < 4) return NULL;
    const uint32_t c0 = get32(buf);
    uint32_t n;
    int has_run;
    const uint8_t* run_flags = NULL;
    uint64_t pos;
    if ((c0 & 0xFFFFu) == PORTABLE_COOKIE) {
        has_run = 1;
        n = (c0 >> 16) + 1u;
        run_flags = buf + 4;
        pos = 4u + (n + 7u) / 8u;
    } else if (c0 == PORTABLE_COOKIE_NO_RUN) {
        if (len < 8) return NULL;
        has_run = 0;
        n = get32(buf + 4);
        if (n > 65536u) return NULL;
        pos = 8;
    } else {
        return NULL;
    }
    if (pos + 4ull * n > len) return NULL;
    const uint8_t* hdr = buf + pos;
    pos += 4ull * n;
    if (!has_run || n >= PORTABLE_NO_OFFSET_THRESHOLD) pos += 4ull * n;
    if (pos > len) return NULL;
    rl_bitmap* b = rl_create();
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t key = get16(hdr + 4u * i);
        const uint32_t card = get16(hdr + 4u * i + 2u) + 1u;
        if (i > 0 && key <= b->keys[b->n - 1]) goto bad;
        if (has_run && (run_flags[i / 8u] >> (i % 8u)) & 1u) {
            if (pos + 2 > len) goto bad;
            const uint32_t nr = get16(buf + pos);
            pos += 2;
            if (pos + 4ull * nr > len) goto bad;
            uint16_t* r = (uint16_t*)malloc(4ull * nr + 4);
            for (uint32_t k = 0; k < 2u * nr; ++k) r[k] = (uint16_t)get16(buf + pos + 2ull * k);
            pos += 4ull * nr;
            for (uint32_t k = 0; k < nr; ++k)
                if ((uint32_t)r[2 * k] + r[2 * k + 1] > 0xFFFFu) {
                    free(r);
                    goto bad;
                }
            rl_push(b, (uint16_t)key, ORC_TC_RUN, (int32_t)nr, r);
        } else if (card <= ARRAY_MAX) {
            if (pos + 2ull * card > len) goto bad;
            uint16_t* a = (uint16_t*)malloc(2ull * card);
            for (uint32_t k = 0; k < card; ++k) a[k] = (uint16_t)get16(buf + pos + 2ull * k);
            pos += 2ull * card;
            rl_push(b, (uint16_t)key, ORC_TC_ARRAY, (int32_t)card, a);
        } else {
            if (pos + 8192 > len) goto bad;
            uint64_t* w = (uint64_t*)malloc(8192);
            for (uint32_t k = 0; k < 1024u; ++k)
                w[k] = (uint64_t)get32(buf + pos + 8ull * k) | ((uint64_t)get32(buf + pos + 8ull * k + 4) << 32);
            pos += 8192;
            rl_push(b, (uint16_t)key, ORC_TC_BITSET, (int32_t)card, w);
        }
    }
    if (consumed) *consumed = pos;
    return b;
bad:
    rl_destroy(b);
    return NULL;
}

/*
 * ref_semantics.c -- CPU restatement of the reference's output-layout rules.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Each function follows the cited
 * reference source; quirks are reproduced, not fixed, because bit-exact parity
 * is defined against the reference's behaviour.
 *
 * Pinning (tests/test_oracle_ref.py):
 *   orc_resolve_auto_threshold -- the five verdicts of test/test_promote.cu:257-381
 *                                 and the 4 MiB / per-XCD crossover arithmetic.
 *   orc_upload_from_ids        -- known answers of test/test_promote.cu:183-449 and
 *                                 test/test_complement.cu:129-237; brute-force
 *                                 decode (flat bitset) on random inputs for both the
 *                                 n<=1024 and the n>1024 paths, plus layout
 *                                 invariants (sorted keys, offsets, card clamps).
 *   orc_upload_from_bitset     -- round trip and negation cases of
 *                                 test/test_complement.cu:793-908; brute-force decode.
 *   orc_upload_packed          -- container counts of test/test_upload.cu and
 *                                 test/test_promote.cu:41-165; decode == roaring-lite.
 *   orc_set_operation          -- all 16 DeMorgan combinations (test/test_complement.cu
 *                                 :367-462) and test/test_set_ops.cu cases, checked
 *                                 against a flat-bitset brute force; XOR-identical and
 *                                 disjoint-AND container counts.
 *   orc_multi_and              -- test/test_complement.cu:502-790 cases against a flat
 *                                 bitset AND; the n_containers==1 pin at :644.
 *   orc_contains / decompress  -- exhaustive comparison with a flat bitset built
 *                                 independently from the input IDs.
 *   orc_enumerate_ids          -- the sorted ids of the decoded set (numpy), the
 *                                 total==0 early return on a set_operation result.
 *   orc_promote_to_bitmap      -- test/test_promote.cu:41-150 (counts, decode
 *                                 equality), layout invariants, negation kept
 *                                 (test/test_complement.cu:468-497).
 *   orc_deep_copy              -- field-by-field equality and the pool sizes.
 */
#include "oracle.h"

#include <stdlib.h>
#include <string.h>

#define ORC_OK 0
#define ORC_ERR_ALLOC 1
#define ORC_ERR_INVALID 2

void orc_free(orc_roaring* r)
{
    if (!r) return;
    free(r->keys);
    free(r->types);
    free(r->offsets);
    free(r->cards);
    free(r->bitmap_data);
    free(r->array_data);
    free(r->run_data);
    free(r->key_index);
    memset(r, 0, sizeof(*r));
}

static void* xcalloc(size_t n, size_t sz)
{
    if (n == 0) n = 1;
    return calloc(n, sz);
}

static int cmp_u32(const void* a, const void* b)
{
    uint32_t x = *(const uint32_t*)a, y = *(const uint32_t*)b;
    return (x > y) - (x < y);
}

/* sort + unique in place, returns new length (std::sort + std::unique). */
static uint64_t sort_unique(uint32_t* v, uint64_t n)
{
    if (n == 0) return 0;
    qsort(v, n, sizeof(uint32_t), cmp_u32);
    uint64_t w = 1;
    for (uint64_t i = 1; i < n; ++i)
        if (v[i] != v[w - 1]) v[w++] = v[i];
    return w;
}

static int popc64(uint64_t x) { return __builtin_popcountll(x); }

/* -------------------------------------------------------------------------
 * resolve_auto_threshold -- src/promote.cu:334-367.
 * `l2_bytes` stands in for cudaDeviceGetAttribute(cudaDevAttrL2CacheSize);
 * the reference falls back to 4 MiB when the query fails (:348-352).
 * ------------------------------------------------------------------------- */
uint32_t orc_resolve_auto_threshold(uint32_t universe_size, uint64_t l2_bytes)
{
    if (universe_size == 0) return ORC_PROMOTE_KEEP_DEFAULT;
    uint64_t flat_bytes = ((uint64_t)universe_size + 7u) / 8u;
    if (flat_bytes * 2u > l2_bytes) return ORC_PROMOTE_ALL;
    return ORC_PROMOTE_KEEP_DEFAULT;
}

/* -------------------------------------------------------------------------
 * build_from_device_ids -- src/upload_ids.cu:171-295.
 * Input: sorted unique ids.  Output: all-BITMAP containers, offsets i*8192,
 * card clamp 65536->0 (:105), max_key derived from U (:274-278).
 * ------------------------------------------------------------------------- */
static int build_from_sorted_ids(const uint32_t* u, uint64_t n, uint32_t universe,
                                 orc_roaring* out)
{
    memset(out, 0, sizeof(*out));
    out->universe_size = universe;
    out->total_cardinality = n;
    if (n == 0) return ORC_OK; /* :180-183 */

    /* RLE over the high-16 keys (:185-214). */
    uint32_t n_c = 0;
    for (uint64_t i = 0; i < n; ++i)
        if (i == 0 || (u[i] >> 16) != (u[i - 1] >> 16)) ++n_c;

    out->n_containers = n_c;
    out->n_bitmap_containers = n_c;
    out->keys = (uint16_t*)xcalloc(n_c, 2);
    out->types = (uint8_t*)xcalloc(n_c, 1);
    out->offsets = (uint32_t*)xcalloc(n_c, 4);
    out->cards = (uint16_t*)xcalloc(n_c, 2);
    out->bitmap_pool_words = n_c * 1024u;
    out->bitmap_data = (uint64_t*)xcalloc((size_t)n_c * 1024u, 8);
    if (!out->keys || !out->types || !out->offsets || !out->cards || !out->bitmap_data)
        return ORC_ERR_ALLOC;

    uint32_t c = 0;
    uint64_t run_start = 0;
    for (uint64_t i = 0; i <= n; ++i) {
        if (i == n || (i > run_start && (u[i] >> 16) != (u[run_start] >> 16))) {
            uint64_t count = i - run_start;
            out->keys[c] = (uint16_t)(u[run_start] >> 16);
            out->types[c] = ORC_BITMAP;
            out->offsets[c] = (uint32_t)((uint64_t)c * 1024u * 8u);
            out->cards[c] = (uint16_t)(count > 65535 ? 0 : count);
            uint64_t* dst = out->bitmap_data + (size_t)c * 1024u;
            for (uint64_t j = run_start; j < i; ++j) {
                uint32_t low = u[j] & 0xFFFFu;
                dst[low >> 6] |= 1ull << (low & 63u);
            }
            ++c;
            run_start = i;
        }
    }

    uint32_t max_key32 = (universe == 0) ? 0u : ((universe - 1u) >> 16);
    if (max_key32 > 0xFFFFu) max_key32 = 0xFFFFu;
    out->max_key = max_key32;
    out->key_index_len = max_key32 + 1u;
    out->key_index = (uint16_t*)xcalloc(out->key_index_len, 2);
    if (!out->key_index) return ORC_ERR_ALLOC;
    memset(out->key_index, 0xFF, (size_t)out->key_index_len * 2u);
    for (uint32_t i = 0; i < n_c; ++i) {
        /* The reference writes key_index[keys[i]] unchecked (:80-88); a key above
         * max_key is an out-of-bounds write there.  Report it as invalid input. */
        if (out->keys[i] > max_key32) return ORC_ERR_INVALID;
        out->key_index[out->keys[i]] = (uint16_t)i;
    }
    return ORC_OK;
}

/* gpu_upload -- src/upload_ids.cu:302-416 (n > 1024). */
static int gpu_upload_semantics(const uint32_t* ids, uint32_t n, uint32_t universe,
                                orc_roaring* out)
{
    uint32_t* u = (uint32_t*)malloc((size_t)n * 4u);
    if (!u) return ORC_ERR_ALLOC;
    memcpy(u, ids, (size_t)n * 4u);
    uint64_t n_u = sort_unique(u, n);

    int rc;
    if (n_u > (uint64_t)universe / 2u) { /* strict, :359 */
        /* Complement [0,U) \ S by gap expansion (:361-410).  Requires ids < U. */
        if (u[n_u - 1] >= universe) {
            free(u);
            return ORC_ERR_INVALID;
        }
        uint64_t n_comp = (uint64_t)universe - n_u;
        uint32_t* comp = (uint32_t*)malloc((size_t)(n_comp ? n_comp : 1) * 4u);
        if (!comp) {
            free(u);
            return ORC_ERR_ALLOC;
        }
        uint64_t w = 0, j = 0;
        for (uint64_t v = 0; v < universe; ++v) {
            if (j < n_u && u[j] == v) {
                ++j;
                continue;
            }
            comp[w++] = (uint32_t)v;
        }
        rc = build_from_sorted_ids(comp, n_comp, universe, out);
        out->negated = 1;
        out->total_cardinality = n_u; /* logical count, :408 */
        free(comp);
    } else {
        rc = build_from_sorted_ids(u, n_u, universe, out);
    }
    free(u);
    return rc;
}

/* cpu_upload -- src/upload_ids.cu:421-561 (n <= 1024). */
static int cpu_upload_semantics(const uint32_t* ids, uint32_t n, uint32_t universe,
                                uint32_t eff_thr, orc_roaring* out)
{
    memset(out, 0, sizeof(*out));
    out->universe_size = universe;
    uint32_t* u = (uint32_t*)malloc((size_t)n * 4u);
    if (!u) return ORC_ERR_ALLOC;
    memcpy(u, ids, (size_t)n * 4u);
    uint64_t m = sort_unique(u, n);
    out->total_cardinality = m;

    uint32_t* v = u;
    uint64_t nv = m;
    uint32_t* comp = NULL;
    if (m > (uint64_t)universe / 2u) { /* :437 */
        comp = (uint32_t*)malloc((size_t)(universe ? universe : 1) * 4u);
        if (!comp) {
            free(u);
            return ORC_ERR_ALLOC;
        }
        uint64_t w = 0, j = 0;
        for (uint32_t x = 0; x < universe; ++x) { /* :443-449 */
            if (j < m && u[j] == x) {
                ++j;
            } else {
                comp[w++] = x;
            }
        }
        v = comp;
        nv = w;
        out->negated = 1;
    }
    if (nv == 0) {
        free(u);
        free(comp);
        return ORC_OK; /* :454-456 */
    }

    uint32_t n_c = 0;
    for (uint64_t i = 0; i < nv; ++i)
        if (i == 0 || (v[i] >> 16) != (v[i - 1] >> 16)) ++n_c;
    out->n_containers = n_c;
    out->keys = (uint16_t*)xcalloc(n_c, 2);
    out->types = (uint8_t*)xcalloc(n_c, 1);
    out->offsets = (uint32_t*)xcalloc(n_c, 4);
    out->cards = (uint16_t*)xcalloc(n_c, 2);
    out->bitmap_data = (uint64_t*)xcalloc((size_t)n_c * 1024u, 8);
    out->array_data = (uint16_t*)xcalloc(nv, 2);
    if (!out->keys || !out->types || !out->offsets || !out->cards || !out->bitmap_data ||
        !out->array_data) {
        free(u);
        free(comp);
        return ORC_ERR_ALLOC;
    }
    uint32_t n_bitmap = 0, n_array = 0, bmp_words = 0, arr_elems = 0;
    uint32_t c = 0;
    uint64_t start = 0;
    for (uint64_t i = 0; i <= nv; ++i) {
        if (i == nv || (i > start && (v[i] >> 16) != (v[start] >> 16))) {
            uint32_t card = (uint32_t)(i - start);
            out->keys[c] = (uint16_t)(v[start] >> 16);
            out->cards[c] = (uint16_t)(card > 65535 ? 0 : card); /* :491 */
            if (card > eff_thr) {                                 /* :493 */
                out->types[c] = ORC_BITMAP;
                out->offsets[c] = bmp_words * 8u;
                uint64_t* dst = out->bitmap_data + bmp_words;
                for (uint64_t j = start; j < i; ++j) {
                    uint32_t low = v[j] & 0xFFFFu;
                    dst[low >> 6] |= 1ull << (low & 63u);
                }
                bmp_words += 1024u;
                ++n_bitmap;
            } else {
                out->types[c] = ORC_ARRAY;
                out->offsets[c] = arr_elems * 2u;
                for (uint64_t j = start; j < i; ++j) out->array_data[arr_elems++] = (uint16_t)v[j];
                ++n_array;
            }
            ++c;
            start = i;
        }
    }
    out->n_bitmap_containers = n_bitmap;
    out->n_array_containers = n_array;
    out->bitmap_pool_words = bmp_words;
    if (bmp_words == 0) {
        free(out->bitmap_data);
        out->bitmap_data = NULL;
    }
    if (arr_elems == 0) {
        free(out->array_data);
        out->array_data = NULL;
    } else {
        out->array_pool_bytes = arr_elems * 2u; /* :542 */
    }
    out->max_key = out->keys[n_c - 1]; /* :547 -- last key, not U */
    out->key_index_len = out->max_key + 1u;
    out->key_index = (uint16_t*)xcalloc(out->key_index_len, 2);
    memset(out->key_index, 0xFF, (size_t)out->key_index_len * 2u);
    for (uint32_t i = 0; i < n_c; ++i) out->key_index[out->keys[i]] = (uint16_t)i;
    free(u);
    free(comp);
    return ORC_OK;
}

/* upload_from_ids -- src/upload_ids.cu:567-591. */
int orc_upload_from_ids(const uint32_t* ids, uint32_t n_ids, uint32_t universe_size,
                        uint32_t bitmap_threshold, uint64_t l2_bytes, orc_roaring* out)
{
    uint32_t eff = bitmap_threshold;
    if (bitmap_threshold == ORC_PROMOTE_AUTO) eff = orc_resolve_auto_threshold(universe_size, l2_bytes);
    if (n_ids == 0) {
        memset(out, 0, sizeof(*out));
        out->universe_size = universe_size;
        return ORC_OK;
    }
    if (n_ids > 1024u) return gpu_upload_semantics(ids, n_ids, universe_size, out); /* :585-587 */
    return cpu_upload_semantics(ids, n_ids, universe_size, eff, out);
}

/* -------------------------------------------------------------------------
 * upload_from_bitset / upload_from_device_bitset / build_from_device_bitset
 * -- src/upload_ids.cu:806-893, 704-801, 606-701.
 * ------------------------------------------------------------------------- */
static int build_from_bitset(const uint32_t* w, uint32_t n_words, uint32_t universe, int negate,
                             uint64_t original_card, orc_roaring* out)
{
    memset(out, 0, sizeof(*out));
    uint32_t n_chunks = (uint32_t)(((uint64_t)n_words + 2047u) / 2048u);
    uint32_t* pc = (uint32_t*)xcalloc(n_chunks, 4);
    uint32_t* map = (uint32_t*)xcalloc(n_chunks, 4);
    if (!pc || !map) {
        free(pc);
        free(map);
        return ORC_ERR_ALLOC;
    }
    uint64_t total = 0;
    uint32_t n_c = 0;
    for (uint32_t c = 0; c < n_chunks; ++c) {
        uint32_t s = 0;
        for (uint32_t i = 0; i < 2048u; ++i) {
            uint64_t idx = (uint64_t)c * 2048u + i;
            if (idx < n_words) s += (uint32_t)__builtin_popcount(w[idx]);
        }
        pc[c] = s;
        total += s;
        map[c] = s ? n_c++ : 0xFFFFFFFFu;
    }
    out->universe_size = universe;
    out->total_cardinality = negate ? original_card : total; /* :740 */
    out->negated = negate;
    out->n_containers = n_c;
    out->n_bitmap_containers = n_c;
    if (n_c == 0) {
        free(pc);
        free(map);
        return ORC_OK;
    }
    out->keys = (uint16_t*)xcalloc(n_c, 2);
    out->types = (uint8_t*)xcalloc(n_c, 1);
    out->offsets = (uint32_t*)xcalloc(n_c, 4);
    out->cards = (uint16_t*)xcalloc(n_c, 2);
    out->bitmap_pool_words = n_c * 1024u;
    out->bitmap_data = (uint64_t*)xcalloc((size_t)n_c * 1024u, 8);
    uint32_t last = 0;
    for (uint32_t c = 0; c < n_chunks; ++c) {
        if (map[c] == 0xFFFFFFFFu) continue;
        uint32_t o = map[c];
        uint64_t* dst = out->bitmap_data + (size_t)o * 1024u;
        for (uint32_t i = 0; i < 1024u; ++i) { /* :669-675 */
            uint64_t i0 = (uint64_t)c * 2048u + 2u * i, i1 = i0 + 1;
            uint64_t w0 = i0 < n_words ? w[i0] : 0u, w1 = i1 < n_words ? w[i1] : 0u;
            dst[i] = w0 | (w1 << 32);
        }
        out->keys[o] = (uint16_t)c;
        out->types[o] = ORC_BITMAP;
        out->offsets[o] = o * 8192u;
        out->cards[o] = (uint16_t)(pc[c] > 65535u ? 0 : pc[c]); /* :684 */
        last = c;
    }
    out->max_key = (uint16_t)last; /* :778-785 -- last non-empty chunk */
    out->key_index_len = out->max_key + 1u;
    out->key_index = (uint16_t*)xcalloc(out->key_index_len, 2);
    memset(out->key_index, 0xFF, (size_t)out->key_index_len * 2u);
    for (uint32_t c = 0; c < n_chunks; ++c)
        if (map[c] != 0xFFFFFFFFu && c < out->key_index_len) out->key_index[c] = (uint16_t)map[c];
    free(pc);
    free(map);
    return ORC_OK;
}

int orc_upload_from_bitset(const uint32_t* words, uint32_t n_words, uint32_t universe_size,
                           orc_roaring* out)
{
    if (n_words == 0) { /* :811-815 */
        memset(out, 0, sizeof(*out));
        out->universe_size = universe_size;
        return ORC_OK;
    }
    uint64_t total = 0;
    for (uint32_t i = 0; i < n_words; ++i) total += (uint32_t)__builtin_popcount(words[i]);
    if (total > (uint64_t)universe_size / 2u) { /* :837 */
        uint32_t* inv = (uint32_t*)malloc((size_t)n_words * 4u);
        if (!inv) return ORC_ERR_ALLOC;
        for (uint32_t i = 0; i < n_words; ++i) inv[i] = ~words[i]; /* :848 */
        uint32_t tail_bits = universe_size % 32u;                  /* :851-858 */
        if (tail_bits > 0) {
            uint32_t t = universe_size / 32u;
            if (t < n_words) inv[t] &= (1u << tail_bits) - 1u;
        }
        int rc = build_from_bitset(inv, n_words, universe_size, 1, total, out);
        free(inv);
        return rc;
    }
    return build_from_bitset(words, n_words, universe_size, 0, 0, out);
}

/* -------------------------------------------------------------------------
 * upload(roaring_bitmap_t*) packed layout -- src/upload.cpp:89-316.
 * The caller has already applied the complement of upload(bm, U) (:296-316)
 * when `complement_applied` is set; then negated=true and total=logical_card.
 * ------------------------------------------------------------------------- */
int orc_upload_packed(const orc_container* conts, uint32_t n, uint32_t explicit_universe,
                      int complement_applied, uint64_t logical_card, uint32_t bitmap_threshold,
                      uint64_t l2_bytes, orc_roaring* out)
{
    memset(out, 0, sizeof(*out));
    if (n == 0) { /* :268-272 */
        out->universe_size = explicit_universe;
        if (complement_applied) {
            out->negated = 1;
            out->total_cardinality = logical_card;
        }
        return ORC_OK;
    }
    uint32_t universe = explicit_universe;
    if (universe == 0) universe = ((uint32_t)conts[n - 1].key + 1u) << 16; /* :96-100, wraps */
    uint32_t eff = bitmap_threshold;
    if (eff == ORC_PROMOTE_AUTO) eff = orc_resolve_auto_threshold(universe, l2_bytes);
    int promote_all = eff < ORC_PROMOTE_KEEP_DEFAULT; /* :104 */
    if (promote_all && bitmap_threshold == ORC_PROMOTE_AUTO) { /* :112-118 */
        uint64_t promoted = (uint64_t)n * 1024u * 8u;
        uint64_t bitset = ((uint64_t)universe + 7u) / 8u;
        if (promoted * 2u >= bitset) promote_all = 0;
    }
    uint64_t bmp_words = 0, arr_elems = 0, run_pairs = 0;
    uint32_t n_bitmap = 0, n_array = 0, n_run = 0;
    for (uint32_t i = 0; i < n; ++i) { /* :120-134 */
        if (conts[i].typecode == ORC_TC_BITSET) {
            ++n_bitmap;
            bmp_words += 1024u;
        } else if (conts[i].typecode == ORC_TC_ARRAY) {
            if (promote_all)
                bmp_words += 1024u;
            else {
                ++n_array;
                arr_elems += (uint64_t)conts[i].card;
            }
        } else if (conts[i].typecode == ORC_TC_RUN) {
            if (promote_all)
                bmp_words += 1024u;
            else {
                ++n_run;
                run_pairs += (uint64_t)conts[i].card;
            }
        }
    }
    if (promote_all) {
        n_bitmap = n;
        n_array = 0;
        n_run = 0;
    }
    out->n_containers = n;
    out->n_bitmap_containers = n_bitmap;
    out->n_array_containers = n_array;
    out->n_run_containers = n_run;
    out->universe_size = universe;
    out->max_key = conts[n - 1].key;
    out->key_index_len = out->max_key + 1u;
    out->keys = (uint16_t*)xcalloc(n, 2);
    out->types = (uint8_t*)xcalloc(n, 1);
    out->offsets = (uint32_t*)xcalloc(n, 4);
    out->cards = (uint16_t*)xcalloc(n, 2);
    out->key_index = (uint16_t*)xcalloc(out->key_index_len, 2);
    out->bitmap_pool_words = (uint32_t)bmp_words;
    if (bmp_words) out->bitmap_data = (uint64_t*)xcalloc(bmp_words, 8);
    if (arr_elems) {
        out->array_data = (uint16_t*)xcalloc(arr_elems, 2);
        out->array_pool_bytes = (uint32_t)(arr_elems * 2u);
    }
    if (run_pairs) {
        out->run_data = (uint16_t*)xcalloc(run_pairs * 2u, 2);
        out->run_pool_bytes = (uint32_t)(run_pairs * 4u);
    }
    memset(out->key_index, 0xFF, (size_t)out->key_index_len * 2u);
    uint64_t total_card = 0;
    uint64_t bc = 0, ac = 0, rc = 0;
    for (uint32_t i = 0; i < n; ++i) { /* pack_into_buffer, :155-225 */
        const orc_container* c = &conts[i];
        out->keys[i] = c->key;
        out->key_index[c->key] = (uint16_t)i;
        if (c->typecode == ORC_TC_BITSET) {
            total_card += (uint64_t)c->card;
        } else if (c->typecode == ORC_TC_ARRAY) {
            total_card += (uint64_t)c->card;
        } else {
            const uint16_t* runs = (const uint16_t*)c->data;
            for (int32_t r = 0; r < c->card; ++r) total_card += (uint64_t)runs[2 * r + 1] + 1u;
        }
        if (promote_all) {
            out->types[i] = ORC_BITMAP;
            out->offsets[i] = (uint32_t)(bc * 8u);
            uint64_t* dst = out->bitmap_data + bc;
            if (c->typecode == ORC_TC_BITSET) {
                out->cards[i] = (uint16_t)(c->card > 65535 ? 0 : c->card);
                memcpy(dst, c->data, 8192);
            } else if (c->typecode == ORC_TC_ARRAY) {
                const uint16_t* a = (const uint16_t*)c->data;
                out->cards[i] = (uint16_t)c->card;
                for (int32_t j = 0; j < c->card; ++j) dst[a[j] >> 6] |= 1ull << (a[j] & 63u);
            } else {
                const uint16_t* runs = (const uint16_t*)c->data;
                out->cards[i] = (uint16_t)c->card; /* n_runs, :193 */
                for (int32_t r = 0; r < c->card; ++r) {
                    uint32_t s = runs[2 * r], l = runs[2 * r + 1];
                    for (uint32_t v = s; v <= s + l; ++v) dst[v >> 6] |= 1ull << (v & 63u);
                }
            }
            bc += 1024u;
        } else if (c->typecode == ORC_TC_BITSET) {
            out->types[i] = ORC_BITMAP;
            out->offsets[i] = (uint32_t)(bc * 8u);
            out->cards[i] = (uint16_t)(c->card > 65535 ? 0 : c->card);
            memcpy(out->bitmap_data + bc, c->data, 8192);
            bc += 1024u;
        } else if (c->typecode == ORC_TC_ARRAY) {
            out->types[i] = ORC_ARRAY;
            out->offsets[i] = (uint32_t)(ac * 2u);
            out->cards[i] = (uint16_t)c->card;
            memcpy(out->array_data + ac, c->data, (size_t)c->card * 2u);
            ac += (uint64_t)c->card;
        } else {
            out->types[i] = ORC_RUN;
            out->offsets[i] = (uint32_t)(rc * 4u);
            out->cards[i] = (uint16_t)c->card;
            memcpy(out->run_data + rc * 2u, c->data, (size_t)c->card * 4u);
            rc += (uint64_t)c->card;
        }
    }
    out->total_cardinality = total_card; /* roaring_bitmap_get_cardinality, :238 */
    if (complement_applied) {
        out->negated = 1;
        out->total_cardinality = logical_card; /* :308-310 */
    }
    return ORC_OK;
}

/* -------------------------------------------------------------------------
 * set_operation -- src/set_ops.cu:76-122 (matching), :533-565 (DeMorgan),
 * :567-1207 (classification, slot order, drop rules, assembly).
 * ------------------------------------------------------------------------- */
enum { CAT_BB, CAT_BA, CAT_AA, CAT_MIXED, CAT_COPY_BMP, CAT_COPY_ARR, CAT_COPY_RUN };

typedef struct {
    uint16_t key;
    int32_t ai, bi;
    int cat;
    uint32_t slot; /* bitmap slot, or array/run element offset (u16 units) */
    uint32_t size; /* array elements or run pairs reserved */
} orc_work;

static void resolve_negation(int* op, const orc_roaring** a, const orc_roaring** b, int* neg)
{
    int na = (*a)->negated, nb = (*b)->negated;
    const orc_roaring* t;
    *neg = 0;
    if (!na && !nb) return;
#define SWAP_AB() (t = *a, *a = *b, *b = t)
    switch (*op) {
    case ORC_AND:
        if (na && !nb) {
            *op = ORC_ANDNOT;
            SWAP_AB();
        } else if (!na && nb) {
            *op = ORC_ANDNOT;
        } else {
            *op = ORC_OR;
            *neg = 1;
        }
        break;
    case ORC_OR:
        if (na && !nb) {
            *op = ORC_ANDNOT;
            *neg = 1;
        } else if (!na && nb) {
            *op = ORC_ANDNOT;
            SWAP_AB();
            *neg = 1;
        } else {
            *op = ORC_AND;
            *neg = 1;
        }
        break;
    case ORC_ANDNOT:
        if (na && !nb) {
            *op = ORC_OR;
            *neg = 1;
        } else if (!na && nb) {
            *op = ORC_AND;
        } else {
            *op = ORC_ANDNOT;
            SWAP_AB();
        }
        break;
    case ORC_XOR:
        if (!(na && nb)) *neg = 1;
        break;
    }
#undef SWAP_AB
}

static uint64_t apply_op(int op, uint64_t x, uint64_t y)
{
    switch (op) {
    case ORC_AND: return x & y;
    case ORC_OR: return x | y;
    case ORC_ANDNOT: return x & ~y;
    default: return x ^ y;
    }
}

/* expand_to_bitmap_kernel (:322-368) plus the host bitmap copy (:794-809). */
static void expand_side(const orc_roaring* r, int idx, uint64_t* dst)
{
    memset(dst, 0, 8192);
    uint8_t t = r->types[idx];
    uint32_t off = r->offsets[idx];
    if (t == ORC_BITMAP) {
        memcpy(dst, r->bitmap_data + off / 8u, 8192);
    } else if (t == ORC_ARRAY) {
        const uint16_t* arr = r->array_data + off / 2u;
        for (uint32_t i = 0; i < r->cards[idx]; ++i) dst[arr[i] >> 6] |= 1ull << (arr[i] & 63u);
    } else if (t == ORC_RUN) {
        const uint16_t* runs = r->run_data + off / 2u;
        for (uint32_t k = 0; k < r->cards[idx]; ++k) {
            uint32_t s = runs[2 * k], e = s + runs[2 * k + 1];
            if (e > 0xFFFFu) e = 0xFFFFu;
            for (uint32_t v = s; v <= e; ++v) dst[v >> 6] |= 1ull << (v & 63u);
        }
    }
}

int orc_set_operation(const orc_roaring* a_in, const orc_roaring* b_in, int op, orc_roaring* out)
{
    const orc_roaring* a = a_in;
    const orc_roaring* b = b_in;
    int neg = 0;
    resolve_negation(&op, &a, &b, &neg);
    memset(out, 0, sizeof(*out));
    uint32_t universe = a->universe_size > b->universe_size ? a->universe_size : b->universe_size;

    /* match_containers (:76-122) */
    uint32_t na = a->n_containers, nb = b->n_containers;
    orc_work* work = (orc_work*)xcalloc((size_t)na + nb, sizeof(orc_work));
    if (!work) return ORC_ERR_ALLOC;
    uint32_t nw = 0, ia = 0, ib = 0;
    int keep_a_only = (op == ORC_OR || op == ORC_XOR || op == ORC_ANDNOT);
    int keep_b_only = (op == ORC_OR || op == ORC_XOR);
    while (ia < na || ib < nb) {
        if (ib >= nb || (ia < na && a->keys[ia] < b->keys[ib])) {
            if (keep_a_only) work[nw++] = (orc_work){a->keys[ia], (int32_t)ia, -1, 0, 0, 0};
            ++ia;
        } else if (ia >= na || a->keys[ia] > b->keys[ib]) {
            if (keep_b_only) work[nw++] = (orc_work){b->keys[ib], -1, (int32_t)ib, 0, 0, 0};
            ++ib;
        } else {
            work[nw++] = (orc_work){a->keys[ia], (int32_t)ia, (int32_t)ib, 0, 0, 0};
            ++ia;
            ++ib;
        }
    }
    out->universe_size = universe;
    out->negated = neg;
    if (nw == 0) { /* :588-593 */
        free(work);
        return ORC_OK;
    }

    /* classification (:626-692) */
    uint32_t n_bb = 0, n_ba = 0, n_aa = 0, n_mx = 0, n_cb = 0, n_ca = 0, n_cr = 0;
    for (uint32_t i = 0; i < nw; ++i) {
        orc_work* w = &work[i];
        if (w->ai < 0 || w->bi < 0) {
            uint8_t t = w->ai < 0 ? b->types[w->bi] : a->types[w->ai];
            w->cat = t == ORC_BITMAP ? CAT_COPY_BMP : (t == ORC_ARRAY ? CAT_COPY_ARR : CAT_COPY_RUN);
        } else {
            uint8_t ta = a->types[w->ai], tb = b->types[w->bi];
            if (ta == ORC_BITMAP && tb == ORC_BITMAP)
                w->cat = CAT_BB;
            else if (op == ORC_AND && ((ta == ORC_BITMAP && tb == ORC_ARRAY) ||
                                       (ta == ORC_ARRAY && tb == ORC_BITMAP)))
                w->cat = CAT_BA;
            else if (op == ORC_AND && ta == ORC_ARRAY && tb == ORC_ARRAY)
                w->cat = CAT_AA;
            else
                w->cat = CAT_MIXED;
        }
        switch (w->cat) {
        case CAT_BB: ++n_bb; break;
        case CAT_BA: ++n_ba; break;
        case CAT_AA: ++n_aa; break;
        case CAT_MIXED: ++n_mx; break;
        case CAT_COPY_BMP: ++n_cb; break;
        case CAT_COPY_ARR: ++n_ca; break;
        default: ++n_cr; break;
        }
    }
    uint32_t out_n_bitmap = n_bb + n_mx + n_cb;
    uint32_t out_n_array = n_ba + n_aa + n_ca;
    uint32_t out_n_run = n_cr;

    /* slot / offset assignment (:695-701, :864-886, :1005-1010) */
    uint32_t r_bb = 0, r_mx = 0, r_cb = 0;
    uint64_t ba_tot = 0, aa_tot = 0, ca_tot = 0, cr_pairs = 0;
    for (uint32_t i = 0; i < nw; ++i) {
        orc_work* w = &work[i];
        switch (w->cat) {
        case CAT_BB: w->slot = r_bb++; break;
        case CAT_MIXED: w->slot = n_bb + r_mx++; break;
        case CAT_COPY_BMP: w->slot = n_bb + n_mx + r_cb++; break;
        case CAT_BA: {
            int arr_is_b = a->types[w->ai] == ORC_BITMAP;
            w->size = arr_is_b ? b->cards[w->bi] : a->cards[w->ai];
            w->slot = (uint32_t)ba_tot;
            ba_tot += w->size;
            break;
        }
        default: break;
        }
    }
    for (uint32_t i = 0; i < nw; ++i) {
        orc_work* w = &work[i];
        if (w->cat == CAT_AA) {
            uint32_t ca = a->cards[w->ai], cb = b->cards[w->bi];
            w->size = ca < cb ? ca : cb;
            w->slot = (uint32_t)(ba_tot + aa_tot);
            aa_tot += w->size;
        }
    }
    for (uint32_t i = 0; i < nw; ++i) {
        orc_work* w = &work[i];
        if (w->cat == CAT_COPY_ARR) {
            w->size = w->ai < 0 ? b->cards[w->bi] : a->cards[w->ai];
            w->slot = (uint32_t)(ba_tot + aa_tot + ca_tot);
            ca_tot += w->size;
        } else if (w->cat == CAT_COPY_RUN) {
            w->size = w->ai < 0 ? b->cards[w->bi] : a->cards[w->ai];
            w->slot = (uint32_t)(cr_pairs * 2u);
            cr_pairs += w->size;
        }
    }
    uint64_t total_arr = ba_tot + aa_tot + ca_tot;

    out->n_bitmap_containers = out_n_bitmap;
    out->n_array_containers = out_n_array;
    out->n_run_containers = out_n_run;
    out->bitmap_pool_words = out_n_bitmap * 1024u;
    if (out_n_bitmap) out->bitmap_data = (uint64_t*)xcalloc((size_t)out_n_bitmap * 1024u, 8);
    if (total_arr) out->array_data = (uint16_t*)xcalloc(total_arr, 2);
    out->array_pool_bytes = (uint32_t)(total_arr * 2u);
    if (cr_pairs) out->run_data = (uint16_t*)xcalloc(cr_pairs * 2u, 2);
    out->run_pool_bytes = (uint32_t)(cr_pairs * 4u);
    out->keys = (uint16_t*)xcalloc(nw, 2);
    out->types = (uint8_t*)xcalloc(nw, 1);
    out->offsets = (uint32_t*)xcalloc(nw, 4);
    out->cards = (uint16_t*)xcalloc(nw, 2);
    uint64_t* ta = (uint64_t*)malloc(8192);
    uint64_t* tb = (uint64_t*)malloc(8192);

    /* execution + assembly in work order (:710-1159) */
    uint32_t nc = 0;
    for (uint32_t i = 0; i < nw; ++i) {
        orc_work* w = &work[i];
        switch (w->cat) {
        case CAT_BB:
        case CAT_MIXED: {
            const uint64_t *pa, *pb;
            if (w->cat == CAT_BB) {
                pa = a->bitmap_data + a->offsets[w->ai] / 8u;
                pb = b->bitmap_data + b->offsets[w->bi] / 8u;
            } else {
                expand_side(a, w->ai, ta);
                expand_side(b, w->bi, tb);
                pa = ta;
                pb = tb;
            }
            uint64_t* dst = out->bitmap_data + (size_t)w->slot * 1024u;
            uint32_t pc = 0;
            for (uint32_t k = 0; k < 1024u; ++k) {
                dst[k] = apply_op(op, pa[k], pb[k]);
                pc += (uint32_t)popc64(dst[k]);
            }
            uint16_t card = (uint16_t)(pc > 65535u ? 0 : pc); /* :179-180 */
            if (card == 0 && op != ORC_OR) break;             /* :1111, :1145 */
            out->keys[nc] = w->key;
            out->types[nc] = ORC_BITMAP;
            out->offsets[nc] = w->slot * 8192u;
            out->cards[nc] = card;
            ++nc;
            break;
        }
        case CAT_BA: {
            int bmp_is_a = a->types[w->ai] == ORC_BITMAP;
            const uint64_t* bm = bmp_is_a ? a->bitmap_data + a->offsets[w->ai] / 8u
                                          : b->bitmap_data + b->offsets[w->bi] / 8u;
            const uint16_t* arr = bmp_is_a ? b->array_data + b->offsets[w->bi] / 2u
                                           : a->array_data + a->offsets[w->ai] / 2u;
            /* Emitted in probe order (sorted); the reference's warp-order
             * compaction (:238-246) can permute values inside a container. */
            uint32_t cnt = 0;
            for (uint32_t k = 0; k < w->size; ++k) {
                uint16_t v = arr[k];
                if ((bm[v >> 6] >> (v & 63u)) & 1u) out->array_data[w->slot + cnt++] = v;
            }
            if (cnt == 0) break; /* :1125 */
            out->keys[nc] = w->key;
            out->types[nc] = ORC_ARRAY;
            out->offsets[nc] = w->slot * 2u;
            out->cards[nc] = (uint16_t)cnt;
            ++nc;
            break;
        }
        case CAT_AA: {
            const uint16_t* x = a->array_data + a->offsets[w->ai] / 2u;
            const uint16_t* y = b->array_data + b->offsets[w->bi] / 2u;
            uint32_t cx = a->cards[w->ai], cy = b->cards[w->bi], p = 0, q = 0, cnt = 0;
            while (p < cx && q < cy) { /* :290-304 */
                if (x[p] < y[q])
                    ++p;
                else if (x[p] > y[q])
                    ++q;
                else {
                    out->array_data[w->slot + cnt++] = x[p];
                    ++p;
                    ++q;
                }
            }
            if (cnt == 0) break; /* :1135 */
            out->keys[nc] = w->key;
            out->types[nc] = ORC_ARRAY;
            out->offsets[nc] = w->slot * 2u;
            out->cards[nc] = (uint16_t)cnt;
            ++nc;
            break;
        }
        case CAT_COPY_BMP: {
            const orc_roaring* s = w->ai < 0 ? b : a;
            int si = w->ai < 0 ? w->bi : w->ai;
            memcpy(out->bitmap_data + (size_t)w->slot * 1024u, s->bitmap_data + s->offsets[si] / 8u,
                   8192);
            out->keys[nc] = w->key;
            out->types[nc] = ORC_BITMAP;
            out->offsets[nc] = w->slot * 8192u;
            out->cards[nc] = s->cards[si];
            ++nc;
            break;
        }
        case CAT_COPY_ARR: {
            const orc_roaring* s = w->ai < 0 ? b : a;
            int si = w->ai < 0 ? w->bi : w->ai;
            memcpy(out->array_data + w->slot, s->array_data + s->offsets[si] / 2u,
                   (size_t)w->size * 2u);
            out->keys[nc] = w->key;
            out->types[nc] = ORC_ARRAY;
            out->offsets[nc] = w->slot * 2u;
            out->cards[nc] = (uint16_t)w->size;
            ++nc;
            break;
        }
        default: {
            const orc_roaring* s = w->ai < 0 ? b : a;
            int si = w->ai < 0 ? w->bi : w->ai;
            memcpy(out->run_data + w->slot, s->run_data + s->offsets[si] / 2u, (size_t)w->size * 4u);
            out->keys[nc] = w->key;
            out->types[nc] = ORC_RUN;
            out->offsets[nc] = w->slot * 2u;
            out->cards[nc] = (uint16_t)w->size;
            ++nc;
            break;
        }
        }
    }
    out->n_containers = nc;
    /* total_cardinality, key_index and max_key stay 0 / NULL (:1162-1175). */
    free(ta);
    free(tb);
    free(work);
    return ORC_OK;
}

/* -------------------------------------------------------------------------
 * multi_and -- src/set_ops.cu:1715-1745 (routing) and fused_multi_and_allbitmap
 * :1489-1710 (with kernels :1224-1473).
 * ------------------------------------------------------------------------- */
static int32_t fused_lookup(const orc_roaring* r, uint16_t key)
{
    if (r->n_containers == 0 || r->keys == NULL) return -1;
    uint32_t mkp1 = r->key_index ? r->max_key + 1u : 0u; /* :1614-1617 */
    if (r->key_index && key < mkp1) {
        uint16_t v = r->key_index[key];
        return v == 0xFFFFu ? -1 : (int32_t)v;
    }
    uint32_t lo = 0, hi = r->n_containers; /* :1375-1383 */
    while (lo < hi) {
        uint32_t mid = (lo + hi) >> 1;
        if (r->keys[mid] < key)
            lo = mid + 1;
        else if (r->keys[mid] > key)
            hi = mid;
        else
            return (int32_t)mid;
    }
    return -1;
}

static int fused_multi_and(const orc_roaring* in, uint32_t count, orc_roaring* out)
{
    memset(out, 0, sizeof(*out));
    uint32_t neg_mask = 0;
    for (uint32_t i = 0; i < count && i < 32; ++i)
        if (in[i].negated) neg_mask |= 1u << i;
    uint32_t universe = in[0].universe_size;
    for (uint32_t i = 1; i < count; ++i)
        if (in[i].universe_size > universe) universe = in[i].universe_size;
    uint32_t mkp1 = (uint32_t)(universe + 65535u) / 65536u; /* u32 arithmetic, :1506 */
    if (mkp1 > 65536u) mkp1 = 65536u;
    out->universe_size = universe;

    static uint64_t presence[1024];
    static uint64_t acc[1024];
    uint32_t n_nn = 0;
    for (uint32_t w = 0; w < 1024; ++w) acc[w] = ~0ull;
    for (uint32_t i = 0; i < count; ++i) {
        if (in[i].negated) continue;
        ++n_nn;
        memset(presence, 0, sizeof(presence));
        for (uint32_t c = 0; c < in[i].n_containers; ++c)
            presence[in[i].keys[c] >> 6] |= 1ull << (in[i].keys[c] & 63u);
        for (uint32_t w = 0; w < 1024; ++w) acc[w] &= presence[w];
    }
    if (n_nn == 0) { /* :1253-1263 */
        for (uint32_t w = 0; w < 1024; ++w) {
            uint32_t lo = w * 64u;
            if (lo >= mkp1)
                acc[w] = 0;
            else if (lo + 64u <= mkp1)
                acc[w] = ~0ull;
            else
                acc[w] = (1ull << (mkp1 - lo)) - 1ull;
        }
    }
    uint32_t n_common = 0;
    for (uint32_t w = 0; w < 1024; ++w) n_common += (uint32_t)popc64(acc[w]);
    out->n_containers = n_common;
    out->n_bitmap_containers = n_common;
    if (n_common == 0) return ORC_OK; /* :1579-1583 */

    out->keys = (uint16_t*)xcalloc(n_common, 2);
    out->types = (uint8_t*)xcalloc(n_common, 1);
    out->offsets = (uint32_t*)xcalloc(n_common, 4);
    out->cards = (uint16_t*)xcalloc(n_common, 2);
    out->bitmap_pool_words = n_common * 1024u;
    out->bitmap_data = (uint64_t*)xcalloc((size_t)n_common * 1024u, 8);
    uint32_t k = 0;
    for (uint32_t w = 0; w < 1024; ++w) {
        uint64_t x = acc[w];
        while (x) {
            out->keys[k++] = (uint16_t)(w * 64u + (uint32_t)__builtin_ctzll(x));
            x &= x - 1;
        }
    }
    static const uint64_t zeros[1024];
    uint32_t total = 0; /* u32 atomicAdd target, :1652-1654 */
    for (uint32_t c = 0; c < n_common; ++c) {
        uint64_t* dst = out->bitmap_data + (size_t)c * 1024u;
        for (uint32_t w = 0; w < 1024; ++w) dst[w] = ~0ull;
        for (uint32_t i = 0; i < count; ++i) {
            int32_t idx = fused_lookup(&in[i], out->keys[c]);
            /* Pointer is bitmap_data + idx*1024 (:1390) -- the container index,
             * not its offset. */
            const uint64_t* src = idx < 0 ? zeros : in[i].bitmap_data + (size_t)idx * 1024u;
            int neg = (neg_mask >> i) & 1u;
            for (uint32_t w = 0; w < 1024; ++w) dst[w] &= neg ? ~src[w] : src[w];
        }
        uint32_t pc = 0;
        for (uint32_t w = 0; w < 1024; ++w) pc += (uint32_t)popc64(dst[w]);
        out->cards[c] = (uint16_t)(pc > 65535u ? 65535u : pc); /* clamp, :1468 */
        total += pc;
        out->types[c] = ORC_BITMAP;
        out->offsets[c] = c * 8192u;
    }
    out->max_key = mkp1 == 0 ? 0u : mkp1 - 1u; /* :1687-1688 */
    out->key_index_len = out->max_key + 1u;
    out->key_index = (uint16_t*)xcalloc(out->key_index_len, 2);
    memset(out->key_index, 0xFF, (size_t)out->key_index_len * 2u);
    for (uint32_t c = 0; c < n_common; ++c)
        if (out->keys[c] < out->key_index_len) out->key_index[out->keys[c]] = (uint16_t)c;
    out->total_cardinality = total;
    return ORC_OK;
}

int orc_multi_and(const orc_roaring* inputs, uint32_t count, orc_roaring* out)
{
    memset(out, 0, sizeof(*out));
    if (count == 0) return ORC_OK; /* :1718 */
    if (count == 1) return orc_set_operation(&inputs[0], &inputs[0], ORC_AND, out);
    int all_bitmap = 1;
    for (uint32_t i = 0; i < count; ++i)
        if (inputs[i].n_array_containers > 0 || inputs[i].n_run_containers > 0) all_bitmap = 0;
    if (all_bitmap && count <= 32) return fused_multi_and(inputs, count, out);
    orc_roaring acc, next;
    int rc = orc_set_operation(&inputs[0], &inputs[1], ORC_AND, &acc);
    for (uint32_t i = 2; rc == ORC_OK && i < count; ++i) {
        rc = orc_set_operation(&acc, &inputs[i], ORC_AND, &next);
        orc_free(&acc);
        acc = next;
    }
    *out = acc;
    return rc;
}

/* -------------------------------------------------------------------------
 * GpuRoaringView::contains with make_view -- include/cu_roaring/device/
 * roaring_view.cuh:39-171 and make_view.cuh:9-27.
 * ------------------------------------------------------------------------- */
int orc_contains(const orc_roaring* r, uint32_t id)
{
    uint16_t key = (uint16_t)(id >> 16), low = (uint16_t)(id & 0xFFFFu);
    int neg = r->negated ? 1 : 0;
    int all_bitmap = r->n_array_containers == 0 && r->n_run_containers == 0 && r->key_index != NULL;
    if (all_bitmap) { /* :45-53 */
        if (key > r->max_key) return neg;
        uint16_t idx = r->key_index[key];
        if (idx == 0xFFFFu) return neg;
        uint64_t w = r->bitmap_data[(uint32_t)idx * 1024u + (low >> 6)];
        return (int)((w >> (low & 63u)) & 1u) ^ neg;
    }
    int idx = -1;
    if (r->key_index) { /* lookup_key, :79-87 */
        if (key <= r->max_key) {
            uint16_t v = r->key_index[key];
            idx = v == 0xFFFFu ? -1 : (int)v;
        }
    } else { /* binary_search_keys, :109-123 */
        int lo = 0, hi = (int)r->n_containers - 1;
        while (lo <= hi) {
            int mid = (lo + hi) >> 1;
            if (r->keys[mid] == key) {
                idx = mid;
                break;
            }
            if (r->keys[mid] < key)
                lo = mid + 1;
            else
                hi = mid - 1;
        }
    }
    if (idx < 0) return neg;
    uint32_t off = r->offsets[idx];
    int res = 0;
    switch (r->types[idx]) {
    case ORC_BITMAP: res = (int)((r->bitmap_data[off / 8u + (low >> 6)] >> (low & 63u)) & 1u); break;
    case ORC_ARRAY: {
        const uint16_t* arr = r->array_data + off / 2u;
        int lo = 0, hi = (int)r->cards[idx] - 1;
        while (lo <= hi) {
            int mid = (lo + hi) >> 1;
            if (arr[mid] == low) {
                res = 1;
                break;
            }
            if (arr[mid] < low)
                lo = mid + 1;
            else
                hi = mid - 1;
        }
        break;
    }
    case ORC_RUN: {
        const uint16_t* runs = r->run_data + off / 2u;
        int lo = 0, hi = (int)r->cards[idx] - 1;
        while (lo <= hi) {
            int mid = (lo + hi) >> 1;
            uint32_t s = runs[2 * mid], l = runs[2 * mid + 1];
            if (low < s)
                hi = mid - 1;
            else if (low > s + l)
                lo = mid + 1;
            else {
                res = 1;
                break;
            }
        }
        break;
    }
    default: res = 0;
    }
    return res ^ neg;
}

void orc_contains_many(const orc_roaring* r, const uint32_t* ids, uint64_t n, uint32_t* out)
{
    for (uint64_t i = 0; i < n; ++i) out[i] = (uint32_t)orc_contains(r, ids[i]);
}

/* decompress_to_bitset -- src/decompress.cu:8-151 (bounded to n_words). */
void orc_decompress(const orc_roaring* r, uint32_t* out, uint32_t n_words)
{
    memset(out, 0, (size_t)n_words * 4u);
    for (uint32_t c = 0; c < r->n_containers; ++c) {
        uint32_t key = r->keys[c], base = key * 2048u, off = r->offsets[c];
        if (r->types[c] == ORC_BITMAP) {
            const uint32_t* src = (const uint32_t*)r->bitmap_data + off / 4u;
            for (uint32_t i = 0; i < 2048u; ++i)
                if (base + i < n_words) out[base + i] = src[i];
        } else if (r->types[c] == ORC_ARRAY) {
            const uint16_t* arr = r->array_data + off / 2u;
            for (uint32_t i = 0; i < r->cards[c]; ++i) {
                uint32_t bit = (key << 16) | arr[i];
                if (bit / 32u < n_words) out[bit / 32u] |= 1u << (bit % 32u);
            }
        } else if (r->types[c] == ORC_RUN) {
            const uint16_t* runs = r->run_data + off / 2u;
            for (uint32_t k = 0; k < r->cards[c]; ++k) {
                uint32_t s = runs[2 * k], e = s + runs[2 * k + 1];
                if (e > 0xFFFFu) e = 0xFFFFu;
                for (uint32_t v = s; v <= e; ++v) {
                    uint32_t bit = (key << 16) | v;
                    if (bit / 32u < n_words) out[bit / 32u] |= 1u << (bit % 32u);
                }
            }
        }
    }
    if (r->negated) { /* :128-150 */
        uint32_t full = r->universe_size / 32u, tail = r->universe_size % 32u;
        for (uint32_t i = 0; i < full && i < n_words; ++i) out[i] = ~out[i];
        if (tail > 0 && full < n_words) out[full] ^= (1u << tail) - 1u;
    }
}

/* Logical cardinality of the stored containers (cards wrap at 65536 and RUN
 * cards hold n_runs, so the struct field is not enough). */
uint64_t orc_true_cardinality(const orc_roaring* r)
{
    uint64_t t = 0;
    for (uint32_t c = 0; c < r->n_containers; ++c) {
        uint32_t off = r->offsets[c];
        if (r->types[c] == ORC_BITMAP) {
            const uint64_t* bm = r->bitmap_data + off / 8u;
            for (uint32_t w = 0; w < 1024u; ++w) t += (uint64_t)popc64(bm[w]);
        } else if (r->types[c] == ORC_ARRAY) {
            t += r->cards[c];
        } else {
            const uint16_t* runs = r->run_data + off / 2u;
            for (uint32_t k = 0; k < r->cards[c]; ++k) {
                uint32_t s = runs[2 * k], e = s + runs[2 * k + 1];
                if (e > 0xFFFFu) e = 0xFFFFu;
                t += e - s + 1u;
            }
        }
    }
    return t;
}

/* enumerate_ids -- src/to_csr.cu:161-220.  The stored set's ids in key order
 * as int64; `negated` is ignored (the kernel reads containers only).  Nothing
 * is written when n_containers == 0 or total_cardinality == 0 (:163), so a
 * set_operation result (total left 0, src/set_ops.cu:1162-1175) enumerates
 * nothing.  A bitmap container contributes its set bits; the reference sizes
 * its slice from cardinalities[] (:150-151), which is 0 for a full container
 * (65536 stored as 0) and 65535 for multi_and's clamped one, while its kernel
 * writes every set bit -- an overrun into the next container's slice.  Here a
 * bitmap's count is its popcount, the sorted list the function is for.
 * Returns the number of ids; `out` may be NULL to count only. */
uint64_t orc_enumerate_ids(const orc_roaring* r, int64_t* out)
{
    if (r->n_containers == 0 || r->total_cardinality == 0) return 0;
    uint64_t n = 0;
    for (uint32_t c = 0; c < r->n_containers; ++c) {
        const uint32_t base = (uint32_t)r->keys[c] << 16, off = r->offsets[c];
        if (r->types[c] == ORC_ARRAY) {
            const uint16_t* arr = r->array_data + off / 2u;
            for (uint32_t i = 0; i < r->cards[c]; ++i) {
                if (out) out[n] = (int64_t)(base | arr[i]);
                ++n;
            }
        } else if (r->types[c] == ORC_BITMAP) {
            const uint64_t* bm = r->bitmap_data + off / 8u;
            for (uint32_t w = 0; w < 1024u; ++w)
                for (uint64_t x = bm[w]; x; x &= x - 1) {
                    if (out) out[n] = (int64_t)(base | (w * 64u + (uint32_t)__builtin_ctzll(x)));
                    ++n;
                }
        } else if (r->types[c] == ORC_RUN) {
            const uint16_t* runs = r->run_data + off / 2u;
            for (uint32_t k = 0; k < r->cards[c]; ++k) {
                const uint32_t s = runs[2 * k], len = runs[2 * k + 1];
                for (uint32_t v = 0; v <= len; ++v) {
                    if (out) out[n] = (int64_t)(base | (s + v));
                    ++n;
                }
            }
        }
    }
    return n;
}

static int orc_build_key_index(orc_roaring* out) /* promote.cu:150-158, 307-320 */
{
    if (out->universe_size == 0) return ORC_OK;
    uint32_t mk = (out->universe_size - 1u) >> 16;
    if (mk > 0xFFFFu) mk = 0xFFFFu;
    out->max_key = mk;
    out->key_index_len = mk + 1u;
    out->key_index = (uint16_t*)malloc(sizeof(uint16_t) * out->key_index_len);
    if (!out->key_index) return ORC_ERR_ALLOC;
    memset(out->key_index, 0xFF, sizeof(uint16_t) * out->key_index_len);
    for (uint32_t i = 0; i < out->n_containers; ++i)
        if (out->keys[i] <= mk) out->key_index[out->keys[i]] = (uint16_t)i;
    return ORC_OK;
}

/* promote_to_bitmap -- src/promote.cu:233-323.  Every container becomes a
 * BITMAP at offset i*8192; keys and cardinalities are copied verbatim (a RUN
 * container's card keeps its n_runs); universe, total and negated carry over;
 * max_key and key_index come from the universe (0 / none when it is 0).  With
 * no array or run container the first n x 8 KiB of the bitmap pool are copied
 * as they lie (:268-276).  An empty input gives the all-zero struct (:236). */
int orc_promote_to_bitmap(const orc_roaring* src, orc_roaring* out)
{
    memset(out, 0, sizeof(*out));
    const uint32_t n = src->n_containers;
    if (n == 0) return ORC_OK;
    out->n_containers = n;
    out->n_bitmap_containers = n;
    out->universe_size = src->universe_size;
    out->total_cardinality = src->total_cardinality;
    out->negated = src->negated;
    out->keys = (uint16_t*)malloc(sizeof(uint16_t) * n);
    out->types = (uint8_t*)malloc(n);
    out->offsets = (uint32_t*)malloc(sizeof(uint32_t) * n);
    out->cards = (uint16_t*)malloc(sizeof(uint16_t) * n);
    out->bitmap_pool_words = n * 1024u;
    out->bitmap_data = (uint64_t*)calloc((size_t)n * 1024u, sizeof(uint64_t));
    if (!out->keys || !out->types || !out->offsets || !out->cards || !out->bitmap_data) {
        orc_free(out);
        return ORC_ERR_ALLOC;
    }
    memcpy(out->keys, src->keys, sizeof(uint16_t) * n);
    memcpy(out->cards, src->cards, sizeof(uint16_t) * n);
    const int all_bitmap = src->n_array_containers == 0 && src->n_run_containers == 0;
    for (uint32_t c = 0; c < n; ++c) {
        out->types[c] = ORC_BITMAP;
        out->offsets[c] = c * 8192u;
        uint64_t* dst = out->bitmap_data + (size_t)c * 1024u;
        if (all_bitmap) {
            memcpy(dst, src->bitmap_data + (size_t)c * 1024u, 8192);
        } else if (src->types[c] == ORC_BITMAP) {
            memcpy(dst, src->bitmap_data + src->offsets[c] / 8u, 8192);
        } else if (src->types[c] == ORC_ARRAY) {
            const uint16_t* arr = src->array_data + src->offsets[c] / 2u;
            for (uint32_t i = 0; i < src->cards[c]; ++i) dst[arr[i] / 64u] |= 1ull << (arr[i] % 64u);
        } else {
            const uint16_t* runs = src->run_data + src->offsets[c] / 2u;
            for (uint32_t k = 0; k < src->cards[c]; ++k) {
                uint32_t s = runs[2 * k], e = s + runs[2 * k + 1];
                if (e > 0xFFFFu) e = 0xFFFFu;
                for (uint32_t v = s; v <= e; ++v) dst[v / 64u] |= 1ull << (v % 64u);
            }
        }
    }
    return orc_build_key_index(out);
}

/* gpu_roaring_deep_copy -- src/promote.cu:178-231.  Scalar fields always; for
 * n_containers == 0 nothing else.  The bitmap pool copies n_bitmap x 8 KiB
 * (not the whole pool), the array / run pools their *_pool_bytes, and the
 * key_index (max_key + 1 entries) only when present and the universe is
 * non-zero. */
int orc_deep_copy(const orc_roaring* src, orc_roaring* out)
{
    memset(out, 0, sizeof(*out));
    out->n_containers = src->n_containers;
    out->n_bitmap_containers = src->n_bitmap_containers;
    out->n_array_containers = src->n_array_containers;
    out->n_run_containers = src->n_run_containers;
    out->universe_size = src->universe_size;
    out->total_cardinality = src->total_cardinality;
    out->negated = src->negated;
    out->max_key = src->max_key;
    out->array_pool_bytes = src->array_pool_bytes;
    out->run_pool_bytes = src->run_pool_bytes;
    const uint32_t n = src->n_containers;
    if (n == 0) return ORC_OK;
    out->keys = (uint16_t*)malloc(sizeof(uint16_t) * n);
    out->types = (uint8_t*)malloc(n);
    out->offsets = (uint32_t*)malloc(sizeof(uint32_t) * n);
    out->cards = (uint16_t*)malloc(sizeof(uint16_t) * n);
    if (!out->keys || !out->types || !out->offsets || !out->cards) {
        orc_free(out);
        return ORC_ERR_ALLOC;
    }
    memcpy(out->keys, src->keys, sizeof(uint16_t) * n);
    memcpy(out->types, src->types, n);
    memcpy(out->offsets, src->offsets, sizeof(uint32_t) * n);
    memcpy(out->cards, src->cards, sizeof(uint16_t) * n);
    if (src->bitmap_data && src->n_bitmap_containers > 0) {
        out->bitmap_pool_words = src->n_bitmap_containers * 1024u;
        out->bitmap_data = (uint64_t*)malloc(sizeof(uint64_t) * out->bitmap_pool_words);
        if (!out->bitmap_data) { orc_free(out); return ORC_ERR_ALLOC; }
        memcpy(out->bitmap_data, src->bitmap_data, sizeof(uint64_t) * out->bitmap_pool_words);
    }
    if (src->array_data && src->array_pool_bytes > 0) {
        out->array_data = (uint16_t*)malloc(src->array_pool_bytes);
        if (!out->array_data) { orc_free(out); return ORC_ERR_ALLOC; }
        memcpy(out->array_data, src->array_data, src->array_pool_bytes);
    }
    if (src->run_data && src->run_pool_bytes > 0) {
        out->run_data = (uint16_t*)malloc(src->run_pool_bytes);
        if (!out->run_data) { orc_free(out); return ORC_ERR_ALLOC; }
        memcpy(out->run_data, src->run_data, src->run_pool_bytes);
    }
    if (src->key_index && src->universe_size > 0) {
        out->key_index_len = src->max_key + 1u;
        out->key_index = (uint16_t*)malloc(sizeof(uint16_t) * out->key_index_len);
        if (!out->key_index) { orc_free(out); return ORC_ERR_ALLOC; }
        memcpy(out->key_index, src->key_index, sizeof(uint16_t) * out->key_index_len);
    }
    return ORC_OK;
}

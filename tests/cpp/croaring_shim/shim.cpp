// TEST-ONLY implementation of the CRoaring calls the library's adapters make
// (roaring/roaring.h in this directory), on top of the test oracle's
// roaring-lite.  Each container is held in CRoaring's own struct layout
// (roaring::internal::{array,bitset,run}_container_t) and owns its payload.
#include <cstdlib>
#include <cstring>
#include <vector>

#include "oracle.h"
#include "roaring/containers/array.h"
#include "roaring/containers/bitset.h"
#include "roaring/containers/run.h"
#include "roaring/roaring.h"

using roaring::internal::array_container_t;
using roaring::internal::bitset_container_t;
using roaring::internal::rle16_t;
using roaring::internal::run_container_t;

namespace {

constexpr uint8_t TC_BITSET = 1, TC_ARRAY = 2, TC_RUN = 3;  // CRoaring's type codes

void* new_container(uint8_t tc, int32_t card, const void* data)
{
    if (tc == TC_BITSET) {
        auto* b = static_cast<bitset_container_t*>(std::malloc(sizeof(bitset_container_t)));
        b->cardinality = card;
        b->words = static_cast<uint64_t*>(std::malloc(8192));
        std::memcpy(b->words, data, 8192);
        return b;
    }
    if (tc == TC_ARRAY) {
        auto* a = static_cast<array_container_t*>(std::malloc(sizeof(array_container_t)));
        a->cardinality = card;
        a->capacity = card;
        a->array = static_cast<uint16_t*>(std::malloc(2u * (card ? card : 1)));
        std::memcpy(a->array, data, 2u * card);
        return a;
    }
    auto* r = static_cast<run_container_t*>(std::malloc(sizeof(run_container_t)));
    r->n_runs = card;
    r->capacity = card;
    r->runs = static_cast<rle16_t*>(std::malloc(4u * (card ? card : 1)));
    std::memcpy(r->runs, data, 4u * card);
    return r;
}

void free_container(uint8_t tc, void* c)
{
    if (tc == TC_BITSET) std::free(static_cast<bitset_container_t*>(c)->words);
    else if (tc == TC_ARRAY) std::free(static_cast<array_container_t*>(c)->array);
    else std::free(static_cast<run_container_t*>(c)->runs);
    std::free(c);
}

void payload(uint8_t tc, const void* c, int32_t* card, const void** data)
{
    if (tc == TC_BITSET) {
        *card = static_cast<const bitset_container_t*>(c)->cardinality;
        *data = static_cast<const bitset_container_t*>(c)->words;
    } else if (tc == TC_ARRAY) {
        *card = static_cast<const array_container_t*>(c)->cardinality;
        *data = static_cast<const array_container_t*>(c)->array;
    } else {
        *card = static_cast<const run_container_t*>(c)->n_runs;
        *data = static_cast<const run_container_t*>(c)->runs;
    }
}

roaring_bitmap_t* from_lite(const rl_bitmap* b)
{
    auto* r = static_cast<roaring_bitmap_t*>(std::calloc(1, sizeof(roaring_bitmap_t)));
    roaring_array_t& ra = r->high_low_container;
    const uint32_t n = rl_n_containers(b);
    ra.size = ra.allocation_size = static_cast<int32_t>(n);
    ra.keys = static_cast<uint16_t*>(std::malloc(2u * (n ? n : 1)));
    ra.typecodes = static_cast<uint8_t*>(std::malloc(n ? n : 1));
    ra.containers = static_cast<void**>(std::malloc(sizeof(void*) * (n ? n : 1)));
    for (uint32_t i = 0; i < n; ++i) {
        uint16_t key;
        uint8_t tc;
        int32_t card;
        const void* data;
        rl_container_info(b, i, &key, &tc, &card, &data);
        ra.keys[i] = key;
        ra.typecodes[i] = tc;
        ra.containers[i] = new_container(tc, card, data);
    }
    return r;
}

// The stored values, ascending.
std::vector<uint32_t> values_of(const roaring_bitmap_t* r)
{
    std::vector<uint32_t> v;
    const roaring_array_t& ra = r->high_low_container;
    for (int32_t i = 0; i < ra.size; ++i) {
        const uint32_t base = static_cast<uint32_t>(ra.keys[i]) << 16;
        int32_t card;
        const void* d;
        payload(ra.typecodes[i], ra.containers[i], &card, &d);
        if (ra.typecodes[i] == TC_BITSET) {
            const uint64_t* w = static_cast<const uint64_t*>(d);
            for (uint32_t k = 0; k < 65536u; ++k)
                if ((w[k >> 6] >> (k & 63u)) & 1u) v.push_back(base + k);
        } else if (ra.typecodes[i] == TC_ARRAY) {
            const uint16_t* a = static_cast<const uint16_t*>(d);
            for (int32_t k = 0; k < card; ++k) v.push_back(base + a[k]);
        } else {
            const rle16_t* runs = static_cast<const rle16_t*>(d);
            for (int32_t k = 0; k < card; ++k)
                for (uint32_t x = runs[k].value; x <= static_cast<uint32_t>(runs[k].value) + runs[k].length; ++x)
                    v.push_back(base + x);
        }
    }
    return v;
}

void release(roaring_bitmap_t* r)
{
    roaring_array_t& ra = r->high_low_container;
    for (int32_t i = 0; i < ra.size; ++i) free_container(ra.typecodes[i], ra.containers[i]);
    std::free(ra.keys);
    std::free(ra.typecodes);
    std::free(ra.containers);
    ra = roaring_array_t{};
}

}  // namespace

extern "C" {

uint64_t roaring::api::roaring_bitmap_get_cardinality(const roaring_bitmap_t* r)
{
    uint64_t s = 0;
    const roaring_array_t& ra = r->high_low_container;
    for (int32_t i = 0; i < ra.size; ++i) {
        int32_t card;
        const void* d;
        payload(ra.typecodes[i], ra.containers[i], &card, &d);
        if (ra.typecodes[i] != TC_RUN) {
            s += static_cast<uint64_t>(card);
        } else {
            const rle16_t* runs = static_cast<const rle16_t*>(d);
            for (int32_t k = 0; k < card; ++k) s += runs[k].length + 1u;
        }
    }
    return s;
}

roaring_bitmap_t* roaring::api::roaring_bitmap_copy(const roaring_bitmap_t* r)
{
    auto* c = static_cast<roaring_bitmap_t*>(std::calloc(1, sizeof(roaring_bitmap_t)));
    const roaring_array_t& ra = r->high_low_container;
    roaring_array_t& rc = c->high_low_container;
    const int32_t n = ra.size;
    rc.size = rc.allocation_size = n;
    rc.keys = static_cast<uint16_t*>(std::malloc(2u * (n ? n : 1)));
    rc.typecodes = static_cast<uint8_t*>(std::malloc(n ? n : 1));
    rc.containers = static_cast<void**>(std::malloc(sizeof(void*) * (n ? n : 1)));
    for (int32_t i = 0; i < n; ++i) {
        int32_t card;
        const void* d;
        payload(ra.typecodes[i], ra.containers[i], &card, &d);
        rc.keys[i] = ra.keys[i];
        rc.typecodes[i] = ra.typecodes[i];
        rc.containers[i] = new_container(ra.typecodes[i], card, d);
    }
    return c;
}

void roaring::api::roaring_bitmap_flip_inplace(roaring_bitmap_t* r, uint64_t range_start, uint64_t range_end)
{
    const std::vector<uint32_t> v = values_of(r);
    rl_bitmap* lite = rl_from_sorted_ids(v.data(), v.size());
    rl_bitmap* flipped = rl_flip(lite, range_start, range_end);
    roaring_bitmap_t* f = from_lite(flipped);
    rl_destroy(lite);
    rl_destroy(flipped);
    release(r);
    r->high_low_container = f->high_low_container;
    std::free(f);
}

void roaring::api::roaring_bitmap_free(const roaring_bitmap_t* r)
{
    if (!r) return;
    auto* m = const_cast<roaring_bitmap_t*>(r);
    release(m);
    std::free(m);
}

roaring_bitmap_t* roaring::api::shim_bitmap_of_ids(const uint32_t* ids, uint64_t n, bool run_optimize)
{
    rl_bitmap* lite = rl_from_ids(ids, n);
    if (run_optimize) rl_run_optimize(lite);
    roaring_bitmap_t* r = from_lite(lite);
    rl_destroy(lite);
    return r;
}

}  // extern "C"

/*
 * TEST-ONLY stand-in for CRoaring's <roaring/roaring.h> (v4.x), which is not
 * available in this image.  It declares just what the library's
 * CU_ROARING_WITH_CROARING adapters touch, with CRoaring's public layout:
 *   - roaring_array_t / roaring_bitmap_t (high_low_container: size, keys,
 *     typecodes, containers), the fields the reference reads in
 *     src/upload.cpp:31-53;
 *   - roaring_bitmap_get_cardinality / _copy / _flip_inplace / _free, the
 *     calls in src/upload.cpp:296-311.
 * The functions are implemented in shim.cpp on top of the test oracle's
 * roaring-lite.  shim_bitmap_of_ids() is a test helper, not CRoaring API.
 * A build against a real CRoaring replaces this directory on the include path.
 */
#ifndef CR_TEST_CROARING_SHIM_ROARING_H
#define CR_TEST_CROARING_SHIM_ROARING_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
namespace roaring {
namespace api {
#endif

typedef struct roaring_array_s {
    int32_t size;
    int32_t allocation_size;
    void** containers;
    uint16_t* keys;
    uint8_t* typecodes;
    uint8_t flags;
} roaring_array_t;

typedef struct roaring_bitmap_s {
    roaring_array_t high_low_container;
} roaring_bitmap_t;

uint64_t roaring_bitmap_get_cardinality(const roaring_bitmap_t* r);
roaring_bitmap_t* roaring_bitmap_copy(const roaring_bitmap_t* r);
void roaring_bitmap_flip_inplace(roaring_bitmap_t* r, uint64_t range_start, uint64_t range_end);
void roaring_bitmap_free(const roaring_bitmap_t* r);

/* Test helper: a bitmap of `ids` (any order, duplicates allowed), with
 * roaring-lite's container choices; run_optimize converts to run containers
 * where their serialized form is smaller. */
roaring_bitmap_t* shim_bitmap_of_ids(const uint32_t* ids, uint64_t n, bool run_optimize);

#ifdef __cplusplus
}  // namespace api
}  // namespace roaring
}  // extern "C"
using namespace ::roaring::api;
#endif

#endif

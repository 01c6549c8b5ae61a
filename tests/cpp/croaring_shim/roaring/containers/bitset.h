/* TEST-ONLY stand-in for CRoaring's <roaring/containers/bitset.h> (v4.x):
 * the bitset container's public layout (cardinality, 1024 u64 words). */
#ifndef CR_TEST_CROARING_SHIM_BITSET_H
#define CR_TEST_CROARING_SHIM_BITSET_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
namespace roaring {
namespace internal {
#endif
typedef struct bitset_container_s {
    int32_t cardinality;
    uint64_t* words;
} bitset_container_t;
#ifdef __cplusplus
}  // namespace internal
}  // namespace roaring
}  // extern "C"
#endif
#endif

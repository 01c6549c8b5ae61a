/* TEST-ONLY stand-in for CRoaring's <roaring/containers/array.h> (v4.x):
 * the array container's public layout (cardinality, capacity, values). */
#ifndef CR_TEST_CROARING_SHIM_ARRAY_H
#define CR_TEST_CROARING_SHIM_ARRAY_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
namespace roaring {
namespace internal {
#endif
typedef struct array_container_s {
    int32_t cardinality;
    int32_t capacity;
    uint16_t* array;
} array_container_t;
#ifdef __cplusplus
}  // namespace internal
}  // namespace roaring
}  // extern "C"
#endif
#endif

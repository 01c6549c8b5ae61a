/* TEST-ONLY stand-in for CRoaring's <roaring/containers/run.h> (v4.x):
 * the run container's public layout (n_runs, capacity, (value, length)
 * pairs covering [value, value + length]). */
#ifndef CR_TEST_CROARING_SHIM_RUN_H
#define CR_TEST_CROARING_SHIM_RUN_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
namespace roaring {
namespace internal {
#endif
typedef struct rle16_s {
    uint16_t value;
    uint16_t length;
} rle16_t;
typedef struct run_container_s {
    int32_t n_runs;
    int32_t capacity;
    rle16_t* runs;
} run_container_t;
#ifdef __cplusplus
}  // namespace internal
}  // namespace roaring
}  // extern "C"
#endif
#endif

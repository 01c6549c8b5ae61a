// Set operations -- counterpart of include/cu_roaring/detail/set_ops.cuh.
#pragma once
#include <hip/hip_runtime_api.h>

#include "cu_roaring/types.hpp"

namespace cu_roaring {

enum class SetOp : uint8_t { AND = 0, OR = 1, ANDNOT = 2, XOR = 3 };

// result = op(a, b); negated inputs are rewritten with DeMorgan.  The caller
// owns the result (free with gpu_roaring_free).
GpuRoaring set_operation(const GpuRoaring& a, const GpuRoaring& b, SetOp op, hipStream_t stream = 0);

// a[0] AND ... AND a[count-1]: fused single pass when every input is
// all-bitmap and count <= 32, else a pairwise chain.
GpuRoaring multi_and(const GpuRoaring* bitmaps, uint32_t count, hipStream_t stream = 0);

}  // namespace cu_roaring

// Fused filtered brute-force top-k (no reference counterpart; see cr_topk_filtered).
#pragma once
#include <hip/hip_runtime_api.h>

#include "cu_roaring/types.hpp"

namespace cu_roaring {

// For each of n_q queries, the k smallest squared L2 distances to the base
// vectors whose id passes `filter` (nullptr = all), ascending, ties by id.
void topk_filtered(const float* d_base, uint64_t n_base, const float* d_queries, uint32_t n_q, uint32_t dim,
                   const GpuRoaring* filter, uint32_t k, float* d_out_dist, int64_t* d_out_ids,
                   hipStream_t stream = 0);

}  // namespace cu_roaring

// Fused filtered brute-force top-k (placeholder until the MFMA kernel lands).
#include "internal.hpp"

using namespace crimpl;

extern "C" int cr_topk_filtered(const float*, uint64_t, const float*, uint32_t, uint32_t, const cr_gpu_roaring*,
                                uint32_t, float*, int64_t*, cr_stream_t)
{
    set_error("cr_topk_filtered: not built yet");
    return CR_ERR_UNSUPPORTED;
}

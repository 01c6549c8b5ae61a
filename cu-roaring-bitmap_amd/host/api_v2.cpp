// Host C++ API of the batch library (namespace cu_roaring::v2) over the C ABI:
// the drop-in surface of the reference's v2/include/cu_roaring_v2/api.hpp.
// Failures throw what the reference throws: std::invalid_argument,
// std::out_of_range, else std::runtime_error.
#include <stdexcept>
#include <string>

#include "cu_roaring_v2/api.hpp"

namespace cu_roaring::v2 {

static cr_stream_t S(hipStream_t s) { return reinterpret_cast<cr_stream_t>(s); }

static void check(int rc, const char* what)
{
    if (rc == CR_OK) return;
    const std::string msg = std::string(what) + ": " + cr_last_error();
    if (rc == CR_ERR_RANGE) throw std::out_of_range(msg);
    if (rc == CR_ERR_INVALID) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

GpuRoaringBatch upload_batch(const HostContainer* const* bitmaps, const uint32_t* n_containers, uint32_t n,
                             hipStream_t stream)
{
    GpuRoaringBatch b;
    check(cr_upload_batch(bitmaps, n_containers, n, S(stream), to_abi(&b)), "upload_batch");
    return b;
}

void free_batch(GpuRoaringBatch& batch) { check(cr_free_batch(to_abi(&batch)), "free_batch"); }

GpuRoaringBatch promote_batch(const GpuRoaringBatch& batch, hipStream_t stream)
{
    GpuRoaringBatch b;
    check(cr_promote_batch(to_abi(&batch), S(stream), to_abi(&b)), "promote_batch");
    return b;
}

GpuRoaringView make_view(const GpuRoaringBatch& batch, uint32_t bitmap_idx)
{
    GpuRoaringView v;
    check(cr_batch_make_view(to_abi(&batch), bitmap_idx, to_abi(&v)), "make_view");
    return v;
}

GpuRoaringBatch multi_and(const GpuRoaringBatch& batch, const uint32_t* input_indices, uint32_t n_inputs,
                          hipStream_t stream)
{
    GpuRoaringBatch b;
    check(cr_batch_multi_and(to_abi(&batch), input_indices, n_inputs, S(stream), to_abi(&b)), "multi_and");
    return b;
}

void decompress_batch(const GpuRoaringBatch& batch, uint64_t* device_bitsets, uint64_t words_each, hipStream_t stream)
{
    check(cr_batch_decompress(to_abi(&batch), device_bitsets, words_each, S(stream)), "decompress_batch");
}

}  // namespace cu_roaring::v2

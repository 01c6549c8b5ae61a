// Device helpers shared by the conversion and serialization kernels: the
// 2048-word image of one container built in LDS.
//
// Array and run containers are expanded into the image; a run sets its head
// and tail words with ds_or and marks the whole words between them in a
// difference array, whose prefix sum then fills them, so a long run costs the
// workgroup O(1) per run plus one pass over the 2048 words.
#pragma once
#include "internal.hpp"

namespace crimpl {

constexpr int CV_NT = 256;            // threads of every conversion workgroup
constexpr int CV_WPT = 2048 / CV_NT;  // image words per thread (8)

struct alignas(16) Image {
    uint32_t w[2048];
    int32_t cover[2048];
};

__device__ __forceinline__ uint32_t bit_span(uint32_t lo, uint32_t hi)  // bits lo..hi of a word, lo <= hi < 32
{
    const uint32_t n = hi - lo + 1u;
    return (n == 32u ? ~0u : ((1u << n) - 1u)) << lo;
}

// Builds container data (ARRAY values or RUN pairs, `card` of them) into
// img->w; every thread of the workgroup calls it.  Run ends are clamped to
// 0xFFFF (src/decompress.cu:71-72).
__device__ inline void expand_to_lds(const uint8_t type, const uint16_t* data, uint32_t card, Image* img)
{
    const uint32_t t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < CV_WPT; ++j) {
        img->w[j * CV_NT + t] = 0;
        if (type == CR_RUN) img->cover[j * CV_NT + t] = 0;
    }
    __syncthreads();
    if (type == CR_ARRAY) {
        for (uint32_t i = t; i < card; i += CV_NT) {
            const uint32_t v = data[i];
            atomicOr(&img->w[v >> 5], 1u << (v & 31u));
        }
        __syncthreads();
        return;
    }
    for (uint32_t k = t; k < card; k += CV_NT) {
        const uint32_t s = data[2 * k];
        const uint32_t e = min(0xFFFFu, s + data[2 * k + 1]);
        const uint32_t hw = s >> 5, tw = e >> 5;
        if (hw == tw) {
            atomicOr(&img->w[hw], bit_span(s & 31u, e & 31u));
        } else {
            atomicOr(&img->w[hw], bit_span(s & 31u, 31u));
            atomicOr(&img->w[tw], bit_span(0u, e & 31u));
            if (tw > hw + 1u) {
                atomicAdd(&img->cover[hw + 1u], 1);
                atomicAdd(&img->cover[tw], -1);
            }
        }
    }
    __syncthreads();
    // prefix sum of the difference array: thread t owns words [8t, 8t + 8)
    int32_t c[CV_WPT];
    uint32_t local = 0;
#pragma unroll
    for (int j = 0; j < CV_WPT; ++j) {
        c[j] = img->cover[CV_WPT * t + j];
        local += static_cast<uint32_t>(c[j]);
    }
    __shared__ uint32_t red[CV_NT / 64];
    uint32_t total;
    int32_t run = static_cast<int32_t>(block_excl_scan<CV_NT>(local, red, total));
#pragma unroll
    for (int j = 0; j < CV_WPT; ++j) {
        run += c[j];
        if (run > 0) img->w[CV_WPT * t + j] = ~0u;
    }
    __syncthreads();
}

}  // namespace crimpl

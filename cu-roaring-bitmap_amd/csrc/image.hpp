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

// Builds container data (ARRAY values or RUN pairs, `card` of them) into the
// 2048-word image `w`; every thread of the NT-thread workgroup calls it.  Run
// ends are clamped to 0xFFFF (src/decompress.cu:71-72).  With `cover` (2048
// words) runs go through the difference array; without it (the lean
// one-wavefront kernels, meant for inputs that hold no run containers) a run
// met anyway sets its whole words one by one.
template <int NT>
__device__ inline void expand_img(const uint8_t type, const uint16_t* data, uint32_t card, uint32_t* w, int32_t* cover)
{
    constexpr int WPT = 2048 / NT;
    const uint32_t t = threadIdx.x;
    const bool diff = type == CR_RUN && cover != nullptr;
#pragma unroll
    for (int j = 0; j < WPT; ++j) {
        w[j * NT + t] = 0;
        if (diff) cover[j * NT + t] = 0;
    }
    __syncthreads();
    if (type == CR_ARRAY) {
        // eight values a thread loaded before any is set: one load latency per
        // 8 NT values rather than one per NT
        for (uint32_t i0 = t; i0 < card; i0 += 8u * NT) {
            uint32_t v[8];
#pragma unroll
            for (uint32_t k = 0; k < 8u; ++k) {
                const uint32_t i = i0 + k * NT;
                v[k] = i < card ? static_cast<uint32_t>(data[i]) : 0xFFFFFFFFu;
            }
#pragma unroll
            for (uint32_t k = 0; k < 8u; ++k)
                if (v[k] != 0xFFFFFFFFu) atomicOr(&w[v[k] >> 5], 1u << (v[k] & 31u));
        }
        __syncthreads();
        return;
    }
    for (uint32_t k = t; k < card; k += NT) {
        const uint32_t s = data[2 * k];
        const uint32_t e = min(0xFFFFu, s + data[2 * k + 1]);
        const uint32_t hw = s >> 5, tw = e >> 5;
        if (hw == tw) {
            atomicOr(&w[hw], bit_span(s & 31u, e & 31u));
        } else {
            atomicOr(&w[hw], bit_span(s & 31u, 31u));
            atomicOr(&w[tw], bit_span(0u, e & 31u));
            if (diff) {
                if (tw > hw + 1u) {
                    atomicAdd(&cover[hw + 1u], 1);
                    atomicAdd(&cover[tw], -1);
                }
            } else {
                for (uint32_t x = hw + 1u; x < tw; ++x) atomicOr(&w[x], ~0u);
            }
        }
    }
    __syncthreads();
    if (!diff) return;
    // prefix sum of the difference array: thread t owns words [WPT t, WPT t + WPT)
    int32_t c[WPT];
    uint32_t local = 0;
#pragma unroll
    for (int j = 0; j < WPT; ++j) {
        c[j] = cover[WPT * t + j];
        local += static_cast<uint32_t>(c[j]);
    }
    __shared__ uint32_t red[NT / 64];
    uint32_t total;
    int32_t run = static_cast<int32_t>(block_excl_scan<NT>(local, red, total));
#pragma unroll
    for (int j = 0; j < WPT; ++j) {
        run += c[j];
        if (run > 0) w[WPT * t + j] = ~0u;
    }
    __syncthreads();
}

__device__ inline void expand_to_lds(const uint8_t type, const uint16_t* data, uint32_t card, Image* img)
{
    expand_img<CV_NT>(type, data, card, img->w, img->cover);
}

}  // namespace crimpl

// Measurement probe (not part of the library): what bounds the upload's build
// walk.  The library's tile sort (csrc/tiles.hpp) sorts 100M ids over 2^30;
// then, with the packed tiles fresh in the Infinity Cache as in the real call
// (a 512 MiB write evicts it before each tile sort), one of:
//   A  the build's walk, each group's fields XORed into a register (no LDS bits)
//   B  the build's walk with the LDS bit sets (the build minus its write-out)
//   C  a sequential 16-byte read of the same 250 MB of packed tiles
//   T  the tile sort itself
#include <hip/hip_runtime.h>
#include <cstdio>
#include <vector>
#include <algorithm>
#include "tiles.hpp"
using namespace crimpl;
#define CK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("HIP %s at %d\n", hipGetErrorString(e), __LINE__); return 1; } } while (0)

__device__ __forceinline__ uint32_t mix30(uint64_t i) {
    uint64_t x = i * 0x9E3779B97F4A7C15ull; x ^= x >> 29; x *= 0xBF58476D1CE4E5B9ull; x ^= x >> 32;
    return static_cast<uint32_t>(x) & ((1u << 30) - 1u);
}
__global__ void gen(uint32_t* ids, uint32_t n) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) ids[i] = mix30(i % 90000000u);
}

template <bool BITS>
__global__ __launch_bounds__(BUILD_NT) void walk_kernel(const uint32_t* __restrict__ part, const uint16_t* __restrict__ tab,
                                                       IdsGeom g, uint32_t* out) {
    __shared__ alignas(16) uint32_t bits[BK_KEYS * 2048u];
    __shared__ GroupQueue queue;
    __shared__ uint32_t desc[BUILD_WAVES * DESC_CAP];
    const uint32_t t = threadIdx.x;
    const uint32_t b = (blockIdx.x % 8) * build_per_xcd(g.NB) + blockIdx.x / 8;
    if (b >= g.NB) return;
    const uint32_t wave = t >> 6, lane = __lane_id();
    uint32_t acc = 0;
    walk_groups<true>(part, tab, g, b, wave, lane, queue, desc,  // the groups the build walks
        [&] { if (BITS) for (uint32_t i = t; i < BK_KEYS * 512u; i += BUILD_NT) reinterpret_cast<uint4*>(bits)[i] = make_uint4(0,0,0,0); },
        [&](uint32_t, uint32_t, uint32_t n, const uint32_t (&f)[8]) {
            if (n == 0u) return;
#pragma unroll
            for (uint32_t k = 0; k < 8u; ++k) {
                const uint32_t F = f[k] & FIELD_MASK;
                if (BITS) atomicOr(&bits[F >> 5], k < n ? 1u << (F & 31u) : 0u);
                else acc ^= k < n ? F : 0u;
            }
        });
    __syncthreads();
    if (BITS) acc = bits[t * 17];
    if (acc == 0x12345u) out[blockIdx.x] = acc;  // keeps the work
}
__global__ void seq_read(const uint4* __restrict__ p, uint64_t n4, uint32_t* out) {
    uint32_t acc = 0;
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n4; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint4 v = p[i]; acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x12345u) out[0] = acc;
}
__global__ void flushk(uint4* p, uint64_t n4) {
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n4; i += (uint64_t)gridDim.x * blockDim.x) p[i] = make_uint4(1,2,3,4);
}
int main() {
    const uint32_t n = 100000000u;
    IdsGeom g{};
    g.n = n; g.K = 16384; g.NB = 1024; g.n_tiles = (n + TILE - 1) / TILE;
    int dev; hipGetDevice(&dev); int cus; hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    g.G = std::min<uint32_t>(cus, (g.n_tiles + TB - 1) / TB); g.vec = true;
    uint32_t *ids, *part, *gmax, *wgc, *out, *flush; uint16_t* tab; IdsTotals* tot;
    const uint64_t part_words = (uint64_t)g.n_tiles * TILE_WORDS + 8;
    CK(hipMalloc(&ids, n * 4ull)); CK(hipMalloc(&part, part_words * 4)); CK(hipMalloc(&gmax, 4 * g.G));
    CK(hipMalloc(&wgc, 4ull * g.G * g.NB)); CK(hipMalloc(&out, 1 << 20)); CK(hipMalloc(&tot, sizeof(IdsTotals)));
    CK(hipMalloc(&tab, 2ull * ((g.n_tiles + TB - 1) / TB) * TB * (g.NB + 1))); CK(hipMalloc(&flush, 512ull << 20));
    gen<<<4096, 256>>>(ids, n); CK(hipDeviceSynchronize());
    hipEvent_t e0, e1, e2; hipEventCreate(&e0); hipEventCreate(&e1); hipEventCreate(&e2);
    const char* names[] = {"A walk loads only", "B walk + LDS bits", "C sequential read"};
    for (int v = 0; v < 3; ++v) {
        std::vector<float> ts, tw;
        for (int r = 0; r < 7; ++r) {
            flushk<<<cus * 8, 256>>>(reinterpret_cast<uint4*>(flush), (512ull << 20) / 16);
            hipEventRecord(e0);
            ids_tile_sort<false><<<g.G, TS_NT>>>(ids, g, part, tab, gmax, tot, nullptr, wgc);
            hipEventRecord(e1);
            if (v == 0) walk_kernel<false><<<build_grid(g.NB), BUILD_NT>>>(part, tab, g, out);
            else if (v == 1) walk_kernel<true><<<build_grid(g.NB), BUILD_NT>>>(part, tab, g, out);
            else seq_read<<<cus * 8, 256>>>(reinterpret_cast<const uint4*>(part), (uint64_t)g.n_tiles * TILE_WORDS / 4, out);
            hipEventRecord(e2); CK(hipEventSynchronize(e2));
            float a, b; hipEventElapsedTime(&a, e0, e1); hipEventElapsedTime(&b, e1, e2);
            if (r) { ts.push_back(a); tw.push_back(b); }
        }
        std::sort(ts.begin(), ts.end()); std::sort(tw.begin(), tw.end());
        printf("%-22s tile sort %.1f us   this kernel %.1f us   (%.0f GB/s of %.0f MB packed tiles)\n", names[v], ts[3] * 1e3, tw[3] * 1e3,
               part_words * 4 / (tw[3] * 1e-3) / 1e9, part_words * 4 / 1e6);
    }
    return 0;
}

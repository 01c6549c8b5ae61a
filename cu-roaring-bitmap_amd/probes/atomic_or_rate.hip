// Measurement probe (not part of the library): the rate of random global
// atomicOr into a 2^30-bit (128 MiB) bitmap on one MI355X, 100M ids -- the
// one-pass upload design (zero the pool, one device atomic per id, popcount).
// Each variant is timed after a 512 MiB write that evicts the Infinity Cache.
// Every index is id >> 5 (or >> 6), below 2^25 (2^24) words: in bounds.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
#include <vector>
#include <algorithm>
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ldnt(const uint4* p) { const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p)); return make_uint4(v.x, v.y, v.z, v.w); }
#define CK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("HIP %s at %d\n", hipGetErrorString(e), __LINE__); return 1; } } while (0)

__device__ __forceinline__ uint32_t mix30(uint64_t i) {
    uint64_t x = i * 0x9E3779B97F4A7C15ull; x ^= x >> 29; x *= 0xBF58476D1CE4E5B9ull; x ^= x >> 32;
    return static_cast<uint32_t>(x) & ((1u << 30) - 1u);
}
__global__ void gen(uint32_t* ids, uint32_t n) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) ids[i] = mix30(i % 90000000u);
}
__global__ void zero(uint4* p, uint64_t n4) {
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n4; i += (uint64_t)gridDim.x * blockDim.x) p[i] = make_uint4(0,0,0,0);
}
// A: one id per thread per step, u32 atomics, no return
__global__ void orA(const uint32_t* __restrict__ ids, uint32_t n, uint32_t* bm) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const uint32_t id = ids[i];
        __hip_atomic_fetch_or(bm + (id >> 5), 1u << (id & 31), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}
// B: 4 ids a thread (16-B loads), u32 atomics
__global__ void orB(const uint4* __restrict__ ids4, uint32_t n4, uint32_t* bm) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += gridDim.x * blockDim.x) {
        const uint4 v = ldnt(ids4 + i);
        const uint32_t a[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; ++k)
            __hip_atomic_fetch_or(bm + (a[k] >> 5), 1u << (a[k] & 31), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}
// C: 4 ids a thread, u64 atomics
__global__ void orC(const uint4* __restrict__ ids4, uint32_t n4, unsigned long long* bm) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += gridDim.x * blockDim.x) {
        const uint4 v = ldnt(ids4 + i);
        const uint32_t a[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; ++k)
            __hip_atomic_fetch_or(bm + (a[k] >> 6), 1ull << (a[k] & 63), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}
// D: workgroup-scope atomics (not coherent across XCDs: a speed reference only; result may lose bits)
__global__ void orD(const uint4* __restrict__ ids4, uint32_t n4, uint32_t* bm) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += gridDim.x * blockDim.x) {
        const uint4 v = ldnt(ids4 + i);
        const uint32_t a[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; ++k)
            __hip_atomic_fetch_or(bm + (a[k] >> 5), 1u << (a[k] & 31), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
}
// popcount per 8 KiB container (2048 words), one workgroup of 256 per container
__global__ void pc(const uint4* __restrict__ bm4, uint32_t* cnt) {
    const uint4* p = bm4 + (uint64_t)blockIdx.x * 512;
    uint32_t c = 0;
    for (int j = threadIdx.x; j < 512; j += 256) { const uint4 v = p[j]; c += __popc(v.x) + __popc(v.y) + __popc(v.z) + __popc(v.w); }
    __shared__ uint32_t s[256]; s[threadIdx.x] = c; __syncthreads();
    for (int o = 128; o > 0; o >>= 1) { if (threadIdx.x < o) s[threadIdx.x] += s[threadIdx.x + o]; __syncthreads(); }
    if (threadIdx.x == 0) cnt[blockIdx.x] = s[0];
}
int main() {
    const uint32_t n = 100000000u;
    const uint64_t words = 1ull << 25;
    uint32_t *ids, *bm, *cnt, *flush;
    CK(hipMalloc(&ids, n * 4ull)); CK(hipMalloc(&bm, words * 4)); CK(hipMalloc(&cnt, 16384 * 4)); CK(hipMalloc(&flush, 512ull << 20));
    gen<<<4096, 256>>>(ids, n); CK(hipDeviceSynchronize());
    hipEvent_t e0, e1, e2; hipEventCreate(&e0); hipEventCreate(&e1); hipEventCreate(&e2);
    std::vector<uint32_t> hc(16384);
    int dev; hipGetDevice(&dev); int cus; hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    const char* names[] = {"A u32 1/thr", "B u32 4/thr", "C u64 4/thr", "D wg-scope(ref)"};
    for (int variant = 0; variant < 4; ++variant) {
      for (int gmul : {4, 16, 64}) {
        std::vector<float> tz, ta, tp;
        for (int rep = 0; rep < 6; ++rep) {
            zero<<<cus * 8, 256>>>(reinterpret_cast<uint4*>(flush), (512ull << 20) / 16);  // evict MALL
            hipEventRecord(e0);
            zero<<<cus * 8, 256>>>(reinterpret_cast<uint4*>(bm), words / 4);
            hipEventRecord(e1);
            const unsigned g = cus * gmul;
            if (variant == 0) orA<<<g, 256>>>(ids, n, bm);
            else if (variant == 1) orB<<<g, 256>>>(reinterpret_cast<const uint4*>(ids), n / 4, bm);
            else if (variant == 2) orC<<<g, 256>>>(reinterpret_cast<const uint4*>(ids), n / 4, reinterpret_cast<unsigned long long*>(bm));
            else orD<<<g, 256>>>(reinterpret_cast<const uint4*>(ids), n / 4, bm);
            hipEventRecord(e2);
            CK(hipEventSynchronize(e2));
            float a, b; hipEventElapsedTime(&a, e0, e1); hipEventElapsedTime(&b, e1, e2);
            hipEventRecord(e0); pc<<<16384, 256>>>(reinterpret_cast<const uint4*>(bm), cnt); hipEventRecord(e1); CK(hipEventSynchronize(e1));
            float c; hipEventElapsedTime(&c, e0, e1);
            if (rep) { tz.push_back(a); ta.push_back(b); tp.push_back(c); }
        }
        CK(hipMemcpy(hc.data(), cnt, 16384 * 4, hipMemcpyDeviceToHost));
        uint64_t tot = 0; for (auto x : hc) tot += x;
        std::sort(tz.begin(), tz.end()); std::sort(ta.begin(), ta.end()); std::sort(tp.begin(), tp.end());
        printf("%-16s grid=%5d  zero %.1f us  atomics %.1f us (%.2f Gatom/s)  popcount %.1f us  total bits %llu\n", names[variant], cus * gmul,
               tz[2] * 1e3, ta[2] * 1e3, n / (ta[2] * 1e-3) / 1e9, tp[2] * 1e3, (unsigned long long)tot);
      }
    }
    return 0;
}

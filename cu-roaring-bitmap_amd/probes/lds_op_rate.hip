// Measurement probe (not part of the library): LDS operation rates on gfx950.
// Each thread of a 1024-lane (or two 512-lane) workgroup per CU does K random
// LDS operations into an array of S words (every address below S); the time is
// scaled to 100M lane-operations, the work of one 100M-id upload per random
// operation an id needs.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
#include <vector>
#include <algorithm>
#define CK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("HIP %s at %d\n", hipGetErrorString(e), __LINE__); return 1; } } while (0)

enum { OR_NR = 0, OR_RTN, ADD_RTN, WRITE, WRITE_B64_OR, READ, OR_B64, WRITE_SORTEDISH };
template <int OP, uint32_t LOG_S, int NT, int K>
__global__ __launch_bounds__(NT) void probe(uint32_t* out, uint32_t seed) {
    __shared__ uint32_t lds[1u << LOG_S];
    for (uint32_t i = threadIdx.x; i < (1u << LOG_S); i += NT) lds[i] = 0;
    __syncthreads();
    uint32_t x = (blockIdx.x * NT + threadIdx.x) * 0x9E3779B1u ^ seed;
    uint32_t acc = 0;
#pragma unroll 8
    for (int k = 0; k < K; ++k) {
        x = x * 1664525u + 1013904223u;
        const uint32_t a = x >> (32 - LOG_S);
        if (OP == OR_NR) __hip_atomic_fetch_or(&lds[a], 1u << (x & 31), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        else if (OP == OR_RTN) acc += __hip_atomic_fetch_or(&lds[a], 1u << (x & 31), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        else if (OP == ADD_RTN) acc += __hip_atomic_fetch_add(&lds[a], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        else if (OP == WRITE) lds[a] = x;
        else if (OP == READ) acc += lds[a];
        else if (OP == OR_B64) __hip_atomic_fetch_or(reinterpret_cast<unsigned long long*>(lds) + (a >> 1), 1ull << (x & 63), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    __syncthreads();
    if (threadIdx.x < 64) out[blockIdx.x * 64 + threadIdx.x] = lds[threadIdx.x * 7] + acc;
    else if (acc == 0x12345678u) out[0] = acc;
}
template <int OP, uint32_t LOG_S, int NT, int K>
float run(uint32_t* out, int cus, int per_cu) {
    hipEvent_t e0, e1; hipEventCreate(&e0); hipEventCreate(&e1);
    const int grid = cus * per_cu;
    probe<OP, LOG_S, NT, K><<<grid, NT>>>(out, 1);
    std::vector<float> ts;
    for (int r = 0; r < 5; ++r) {
        hipEventRecord(e0);
        probe<OP, LOG_S, NT, K><<<grid, NT>>>(out, r);
        hipEventRecord(e1); hipEventSynchronize(e1);
        float ms; hipEventElapsedTime(&ms, e0, e1); ts.push_back(ms);
    }
    std::sort(ts.begin(), ts.end());
    const double ops = double(grid) * NT * K;
    return float(ts[2] * 1e3 * (1e8 / ops));  // us per 100M lane-ops
}
int main() {
    int dev; hipGetDevice(&dev); int cus; hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    int clk; hipDeviceGetAttribute(&clk, hipDeviceAttributeClockRate, dev);
    printf("CUs %d clock %d kHz\n", cus, clk);
    uint32_t* out; CK(hipMalloc(&out, 64ull * cus * 64 * 4));
    const char* opn[] = {"ds_or (no rtn)", "ds_or_rtn", "ds_add_rtn", "ds_write_b32", "", "ds_read_b32", "ds_or_b64"};
    // one 1024-lane workgroup per CU (S up to 128 KB), K ops a lane, 8 waves of such per CU over the grid
#define ROW(OP, L) printf("%-16s S=%6u B  1x1024/CU: %7.1f us  2x512/CU(half S): %7.1f us  per 100M ops\n", opn[OP], (1u << L) * 4, \
    run<OP, L, 1024, 256>(out, cus, 4), run<OP, (L) - 1, 512, 256>(out, cus, 8));
    ROW(OR_NR, 15) ROW(OR_NR, 14) ROW(OR_NR, 12) ROW(OR_NR, 10)
    ROW(OR_RTN, 15) ROW(ADD_RTN, 15) ROW(ADD_RTN, 11)
    ROW(WRITE, 15) ROW(WRITE, 14) ROW(WRITE, 12)
    ROW(READ, 15) ROW(READ, 12)
    ROW(OR_B64, 15)
    return 0;
}

// Internal runtime shared by the HIP translation units: error reporting,
// stream-ordered allocation of packed result blocks and scratch, and wave64
// primitives for gfx950.
#pragma once
#include <mutex>
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstdio>

#include "cu_roaring_abi.h"

namespace crimpl {

// ---- errors -------------------------------------------------------------
void set_error(const char* fmt, ...);

#define CR_HIP_RET(expr)                                                                    \
    do {                                                                                    \
        hipError_t e__ = (expr);                                                            \
        if (e__ != hipSuccess) {                                                            \
            ::crimpl::set_error("%s:%d: %s: %s", __FILE__, __LINE__, #expr, hipGetErrorString(e__)); \
            return CR_ERR_HIP;                                                              \
        }                                                                                   \
    } while (0)

#define CR_RET(expr)                  \
    do {                              \
        int rc__ = (expr);            \
        if (rc__ != CR_OK) return rc__; \
    } while (0)

#define CR_LAUNCH_CHECK() CR_HIP_RET(hipGetLastError())

inline hipStream_t as_stream(cr_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// ---- stream-ordered device memory ---------------------------------------
int dev_alloc(void** p, size_t bytes, hipStream_t s);
int dev_free(void* p, hipStream_t s);
// hipStreamSynchronize, timed as the host phase "sync".
int sync_stream(hipStream_t s);

// A 256-byte slot of pinned host memory that kernels write with ordinary
// stores (system-coherent); the host reads it after the stream sync.  The guard
// returns the slot to the library's pool.
constexpr size_t HOST_SLOT_BYTES = 256;
struct HostSlot {
    void* host = nullptr;
    void* dev = nullptr;
    uint32_t id = 0;
};
int host_slot_acquire(HostSlot* out);
void host_slot_release(HostSlot* slot);
struct HostSlotGuard {
    HostSlot slot;
    HostSlotGuard() = default;
    HostSlotGuard(const HostSlotGuard&) = delete;
    HostSlotGuard& operator=(const HostSlotGuard&) = delete;
    ~HostSlotGuard() { host_slot_release(&slot); }
    int acquire() { return host_slot_acquire(&slot); }
    template <class T>
    T* dev() const { return static_cast<T*>(slot.dev); }
    template <class T>
    const volatile T* host() const { return static_cast<const volatile T*>(slot.host); }
};

// Copies `bytes` (<= HOST_SLOT_BYTES through a pinned slot) from device
// memory once the stream reaches this point, then synchronises the stream.
int read_back(void* host, const void* dev, size_t bytes, hipStream_t s);

// Host (pageable) -> device copy, stream-ordered: large copies go through a
// ring of pinned chunks, each filled by a pool of host threads while the
// previous chunks' DMA runs; returns once every chunk is enqueued (the source
// may then be reused).  Small copies use hipMemcpyAsync directly.
int h2d_pageable(void* dst, const void* src, size_t bytes, hipStream_t s);

// Scratch that is released (stream-ordered) when the guard leaves scope.
struct Scratch {
    void* ptr = nullptr;
    hipStream_t stream = nullptr;
    Scratch() = default;
    Scratch(const Scratch&) = delete;
    Scratch& operator=(const Scratch&) = delete;
    ~Scratch() { release(); }
    int alloc(size_t bytes, hipStream_t s)
    {
        stream = s;
        return dev_alloc(&ptr, bytes, s);
    }
    void release()
    {
        if (ptr) dev_free(ptr, stream);
        ptr = nullptr;
    }
    template <class T>
    T* at(size_t byte_offset) const
    {
        return reinterpret_cast<T*>(static_cast<char*>(ptr) + byte_offset);
    }
};

// Carves one allocation into 256-byte aligned sections.
struct Carver {
    size_t total = 0;
    size_t add(size_t bytes)
    {
        size_t off = total;
        total += (bytes + 255) & ~size_t(255);
        return off;
    }
};

// Packed output block of a result GpuRoaring (one allocation, _alloc_base set).
struct OutLayout {
    size_t keys = 0, types = 0, offsets = 0, cards = 0, kidx = 0, bmp = 0, arr = 0, run = 0;
    size_t total = 0;
};
OutLayout plan_out(uint64_t n_meta, uint64_t kidx_len, uint64_t bmp_words, uint64_t arr_elems, uint64_t run_u16);
// Allocates the block and points the struct's arrays into it (sections of size
// 0 leave the pointer null).
int alloc_out(cr_gpu_roaring* out, const OutLayout& L, uint64_t n_meta, uint64_t kidx_len, uint64_t bmp_words,
              uint64_t arr_elems, uint64_t run_u16, hipStream_t s);

void reset(cr_gpu_roaring* r);
int free_async(cr_gpu_roaring* r, hipStream_t s);

// The last step of every producing entry point.  `out` is output-only and was
// reset before the call's work began; a call that fails after allocating part
// of its result releases it on its stream and hands back an empty struct, so
// no failure leaks device memory.
inline int produced(int rc, cr_gpu_roaring* out, hipStream_t s)
{
    if (rc != CR_OK) (void)free_async(out, s);
    return rc;
}

// ---- device helpers -------------------------------------------------------
__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

// Streaming 16-byte load and store: global_load/store_dwordx4 with the `nt`
// (nontemporal) policy.  For data touched once (container payloads, id
// streams) this is what lets gfx950 approach its HBM rate: on MI355X a read
// stream of whole 8 KiB blocks runs at 6.7 TB/s with it and 4.0 TB/s without,
// and a copy at 5.7 against 4.7 TB/s (the store needs the policy too).
// Data read again soon by other waves (metadata, shared cache lines) keeps
// ordinary loads.  So does data that the next kernel of the same call reads
// again and that fits in the 256 MB Infinity Cache (the upload's packed tiles,
// a bitset read twice): nontemporal loads and stores do not allocate there, so
// ordinary stores (or loads) of it, beside nontemporal streams of everything
// else, leave it in that cache for the second read.
typedef uint32_t cr_v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 ld_stream(const uint4* p)
{
    const cr_v4u v = __builtin_nontemporal_load(reinterpret_cast<const cr_v4u*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ void st_stream(uint4* p, uint4 v)
{
    const cr_v4u x = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(x, reinterpret_cast<cr_v4u*>(p));
}

__device__ __forceinline__ void st_stream(int64_t* p, int64_t v) { __builtin_nontemporal_store(v, p); }

__device__ __forceinline__ void st_stream(uint2* p, uint2 v)
{
    __builtin_nontemporal_store(static_cast<uint64_t>(v.x) | (static_cast<uint64_t>(v.y) << 32),
                                reinterpret_cast<uint64_t*>(p));
}

// The wave's own LDS writes are visible to its later LDS reads (its LDS
// operations retire in order); this keeps the compiler from moving them across.
__device__ __forceinline__ void wave_lds_fence()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint32_t wave_sum(uint32_t v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Inclusive scan over a full wave with DPP moves (no lane-index registers):
// shifts by 1, 2, 4, 8 within each row of 16 lanes (lanes without a source
// add the `old` value 0), then row 0's total into row 1 and row 2's into row 3
// (row_bcast:15), then lane 31's prefix into rows 2 and 3 (row_bcast:31).
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v)
{
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x111, 0xF, 0xF, false));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x112, 0xF, 0xF, false));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x114, 0xF, 0xF, false));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x118, 0xF, 0xF, false));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x142, 0xA, 0xF, false));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x143, 0xC, 0xF, false));
    return v;
}

// Block-wide sum; `lds` holds one slot per wave.  All threads get the total.
template <int NT>
__device__ __forceinline__ uint32_t block_sum(uint32_t v, uint32_t* lds)
{
    constexpr int NW = NT / 64;
    v = wave_sum(v);
    const uint32_t w = threadIdx.x >> 6;
    if (__lane_id() == 0) lds[w] = v;
    __syncthreads();
    uint32_t t = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) t += lds[i];
    __syncthreads();
    return t;
}

// Block-wide exclusive scan of one value; returns the prefix, writes the total.
template <int NT>
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* lds, uint32_t& total)
{
    constexpr int NW = NT / 64;
    const uint32_t incl = wave_incl_scan(v);
    const uint32_t w = threadIdx.x >> 6;
    if (__lane_id() == 63) lds[w] = incl;
    __syncthreads();
    uint32_t base = 0, t = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const uint32_t x = lds[i];
        base += (static_cast<uint32_t>(i) < w) ? x : 0u;
        t += x;
    }
    __syncthreads();
    total = t;
    return base + incl - v;
}

// K block-wide exclusive scans: each wave scans its K values with DPP moves
// and lane 63 publishes the wave totals; K * NT/64 threads then turn them into
// per-wave prefixes (and the K block totals), and every thread adds its
// wave's prefix.  `lds` needs 2 K NT/64 + K slots; v[k] becomes value k's
// exclusive prefix and total[k] its block total.
template <int NT, int K>
__device__ __forceinline__ void block_excl_scan_multi(uint32_t (&v)[K], uint32_t* lds, uint32_t (&total)[K])
{
    constexpr int NW = NT / 64;
    static_assert(K * NW <= NT, "one thread per (value, wave)");
    const uint32_t t = threadIdx.x, w = t >> 6;
    uint32_t incl[K];
#pragma unroll
    for (int k = 0; k < K; ++k) incl[k] = wave_incl_scan(v[k]);
    if (__lane_id() == 63) {
#pragma unroll
        for (int k = 0; k < K; ++k) lds[k * NW + w] = incl[k];
    }
    __syncthreads();
    if (t < static_cast<uint32_t>(K * NW)) {  // thread (k, i): the totals of value k's waves before wave i
        const uint32_t k = t / NW, i = t % NW;
        uint32_t pre = 0, all = 0;
#pragma unroll
        for (uint32_t j = 0; j < static_cast<uint32_t>(NW); ++j) {
            const uint32_t x = lds[k * NW + j];
            pre += j < i ? x : 0u;
            all += x;
        }
        lds[K * NW + t] = pre;
        if (i == 0) lds[2 * K * NW + k] = all;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < K; ++k) {
        v[k] = lds[K * NW + k * NW + w] + incl[k] - v[k];
        total[k] = lds[2 * K * NW + k];
    }
    __syncthreads();  // lds may be reused
}

// Ordered compaction helper: exclusive rank of `flag` among the block's lanes
// (ballot per wave, wave counts through LDS).  `lds` needs NT/64 slots.
template <int NT>
__device__ __forceinline__ uint32_t block_flag_rank(bool flag, uint32_t* lds, uint32_t& total)
{
    constexpr int NW = NT / 64;
    const unsigned long long m = __ballot(flag);
    const uint32_t lane = __lane_id();
    const unsigned long long below = lane ? (m & (~0ull >> (64 - lane))) : 0ull;
    const uint32_t w = threadIdx.x >> 6;
    if (lane == 0) lds[w] = static_cast<uint32_t>(__popcll(m));
    __syncthreads();
    uint32_t base = 0, t = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const uint32_t x = lds[i];
        base += (static_cast<uint32_t>(i) < w) ? x : 0u;
        t += x;
    }
    __syncthreads();
    total = t;
    return base + static_cast<uint32_t>(__popcll(below));
}

// lower_bound over a sorted u16 array in global memory.
__device__ __forceinline__ uint32_t lower_bound_u16(const uint16_t* a, uint32_t n, uint32_t key)
{
    uint32_t lo = 0, hi = n;
    while (lo < hi) {
        uint32_t mid = (lo + hi) >> 1;
        if (a[mid] < key)
            lo = mid + 1;
        else
            hi = mid;
    }
    return lo;
}

// lower_bound with a whole wavefront: 64 samples per step (log64 n dependent
// loads instead of log2 n).  Every active lane must call it with the same
// arguments and receives the same result.
__device__ __forceinline__ uint32_t wave_lower_bound_u16(const uint16_t* a, uint32_t n, uint32_t key)
{
    const uint32_t lane = __lane_id();
    uint32_t lo = 0, hi = n;  // the answer lies in [lo, hi]
    while (hi - lo > 64) {
        const uint32_t step = (hi - lo + 63) / 64;
        const uint32_t pos = lo + lane * step;
        const bool less = pos < hi && a[pos] < key;
        const uint32_t cnt = static_cast<uint32_t>(__popcll(__ballot(less)));
        if (cnt == 0) return lo;
        const uint32_t nlo = lo + (cnt - 1) * step + 1;
        hi = min(hi, lo + cnt * step);
        lo = nlo;
    }
    const uint32_t pos = lo + lane;
    const bool less = pos < hi && a[pos] < key;
    return lo + static_cast<uint32_t>(__popcll(__ballot(less)));
}

// Fill kernels (used instead of hipMemsetAsync so the work stays capturable).
__global__ void fill_u16_kernel(uint16_t* p, uint16_t v, uint64_t n);
__global__ void fill_u32_kernel(uint32_t* p, uint32_t v, uint64_t n);
int fill_u16(uint16_t* p, uint16_t v, uint64_t n, hipStream_t s);
int fill_u32(uint32_t* p, uint32_t v, uint64_t n, hipStream_t s);

// ---- per-kernel timing (off unless cr_timing_enable(1)) ---------------------
// Each timed launch records a hipEvent pair on its own stream; cr_timing_report
// synchronises the events and returns per-kernel launch counts and milliseconds.
extern bool g_timing_on;
struct TimedLaunch {
    const char* name;
    hipStream_t stream;
    hipEvent_t start = nullptr;
    TimedLaunch(const char* n, hipStream_t s);
    ~TimedLaunch();
};
#define CR_TIMED(name, stream) ::crimpl::TimedLaunch cr_timed_launch__(name, stream)

// Host wall-clock phases (allocation, synchronisation), reported as "host:<name>".
void record_host_ms(const char* name, double ms);
struct HostPhase {
    const char* name;
    double t0;
    explicit HostPhase(const char* n);
    ~HostPhase();
};
#define CR_HOST_PHASE(name) ::crimpl::HostPhase cr_host_phase__(name)

// Grow-only pinned staging buffer, serialised by its mutex; a call that uses
// it synchronises its stream before releasing the lock.
struct PinnedStage {
    std::mutex mu;
    void* ptr = nullptr;
    size_t cap = 0;
    int reserve(size_t bytes)
    {
        if (bytes <= cap) return CR_OK;
        if (ptr) (void)hipHostFree(ptr);
        ptr = nullptr;
        cap = 0;
        const size_t want = bytes > (size_t(1) << 20) ? bytes : (size_t(1) << 20);
        if (hipHostMalloc(&ptr, want, hipHostMallocDefault) != hipSuccess) {
            ptr = nullptr;
            set_error("hipHostMalloc(%zu) failed", want);
            return CR_ERR_ALLOC;
        }
        cap = want;
        return CR_OK;
    }
};

// Up to eight device byte ranges copied by one kernel launch.
struct CopySeg {
    const void* src;
    void* dst;
    uint64_t bytes;
};
struct CopyList {
    CopySeg seg[8];
    uint32_t n;
    uint32_t blk0[9];  // copy_segments: first workgroup of each segment (filled there)
};
int copy_segments(const CopyList& L, hipStream_t s);

// out = exclusive prefix sums of in[0, n) (n <= 65536; in and out distinct).
int scan_exclusive_u64(const uint64_t* in, uint32_t n, uint64_t* out, hipStream_t s);

uint64_t device_l2_bytes(int device);
// Compute units of the current device (cached per device).
uint32_t num_cus();
uint32_t resolve_auto_threshold(uint32_t universe_size, int device);

}  // namespace crimpl

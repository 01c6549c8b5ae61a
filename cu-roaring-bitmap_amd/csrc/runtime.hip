// Runtime pieces shared by every entry point: error state, allocation of
// packed result blocks, free, AUTO threshold, and small utility entry points.
#include <algorithm>
#include <chrono>
#include <condition_variable>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "internal.hpp"

namespace crimpl {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...)
{
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

int sync_stream(hipStream_t s)
{
    CR_HOST_PHASE("sync");
    CR_HIP_RET(hipStreamSynchronize(s));
    return CR_OK;
}

// Read-back slots: 256-byte pieces of pinned host memory that a call's last
// kernel writes its totals into, so the host reads them after the stream sync
// with no copy command (a pageable 24-byte device-to-host copy adds ~11 us to
// a sync on MI355X, a pinned one ~3.5 us, a kernel's own store ~0.2 us).
// Blocks of 256 slots are allocated on demand and kept until the process ends.
static std::mutex g_slot_mu;
static std::vector<char*> g_slot_blocks;
static std::vector<uint32_t> g_slot_free;  // free slot ids: block * 256 + index
constexpr uint32_t SLOTS_PER_BLOCK = 256;

int host_slot_acquire(HostSlot* out)
{
    std::lock_guard<std::mutex> lk(g_slot_mu);
    if (g_slot_free.empty()) {
        void* blk = nullptr;
        if (hipHostMalloc(&blk, SLOTS_PER_BLOCK * HOST_SLOT_BYTES, hipHostMallocDefault) != hipSuccess || !blk) {
            set_error("hipHostMalloc of %u read-back slots failed", SLOTS_PER_BLOCK);
            return CR_ERR_ALLOC;
        }
        const uint32_t b = static_cast<uint32_t>(g_slot_blocks.size());
        g_slot_blocks.push_back(static_cast<char*>(blk));
        for (uint32_t i = SLOTS_PER_BLOCK; i-- > 0;) g_slot_free.push_back(b * SLOTS_PER_BLOCK + i);
    }
    const uint32_t id = g_slot_free.back();
    g_slot_free.pop_back();
    out->id = id;
    out->host = g_slot_blocks[id / SLOTS_PER_BLOCK] + (id % SLOTS_PER_BLOCK) * HOST_SLOT_BYTES;
    void* dev = nullptr;
    if (hipHostGetDevicePointer(&dev, out->host, 0) != hipSuccess || !dev) {
        g_slot_free.push_back(id);
        set_error("hipHostGetDevicePointer failed for a read-back slot");
        return CR_ERR_HIP;
    }
    out->dev = dev;
    return CR_OK;
}

void host_slot_release(HostSlot* slot)
{
    if (!slot->host) return;
    std::lock_guard<std::mutex> lk(g_slot_mu);
    g_slot_free.push_back(slot->id);
    slot->host = nullptr;
    slot->dev = nullptr;
}

int read_back(void* host, const void* dev, size_t bytes, hipStream_t s)
{
    if (bytes > HOST_SLOT_BYTES) {
        CR_HIP_RET(hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, s));
        return sync_stream(s);
    }
    HostSlotGuard hs;
    CR_RET(hs.acquire());
    CR_HIP_RET(hipMemcpyAsync(hs.slot.host, dev, bytes, hipMemcpyDeviceToHost, s));
    CR_RET(sync_stream(s));
    std::memcpy(host, hs.slot.host, bytes);
    return CR_OK;
}

// ---- pageable host -> device copies -----------------------------------------
// A pageable source cannot be DMA'd directly (and registering it is not
// available here), so it is copied into pinned chunks first.  A pool of host
// threads fills chunk i + 1 while chunk i's DMA runs; R chunks rotate, each
// reused only after the event of its previous DMA.  The pool and the ring live
// for the process (never freed: worker threads may still wait on them at exit).
namespace {
constexpr size_t H2D_CHUNK = size_t(16) << 20;
constexpr int H2D_RING = 4;
constexpr size_t H2D_DIRECT = size_t(8) << 20;  // below this, hipMemcpyAsync's own staging

struct CopyPool {
    std::mutex m;
    std::condition_variable cv, done;
    uint64_t gen = 0;
    int pending = 0;
    int workers = 0;
    const char* src = nullptr;
    char* dst = nullptr;
    size_t n = 0;

    void part(int i, int parts)
    {
        const size_t lo = n * static_cast<size_t>(i) / parts, hi = n * static_cast<size_t>(i + 1) / parts;
        if (hi > lo) std::memcpy(dst + lo, src + lo, hi - lo);
    }
    void worker(int i)
    {
        uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> lk(m);
                cv.wait(lk, [&] { return gen != seen; });
                seen = gen;
            }
            part(i + 1, workers + 1);  // the caller copies part 0
            std::lock_guard<std::mutex> lk(m);
            if (--pending == 0) done.notify_one();
        }
    }
    // Copies n bytes with the workers and the calling thread.
    void copy(char* d, const char* s_, size_t bytes)
    {
        {
            std::lock_guard<std::mutex> lk(m);
            dst = d;
            src = s_;
            n = bytes;
            pending = workers;
            ++gen;
        }
        cv.notify_all();
        part(0, workers + 1);
        std::unique_lock<std::mutex> lk(m);
        done.wait(lk, [&] { return pending == 0; });
    }
};

struct H2dRing {
    std::mutex mu;  // one staged copy at a time
    CopyPool* pool = nullptr;
    char* chunk[H2D_RING] = {};
    hipEvent_t ev[H2D_RING] = {};
    bool used[H2D_RING] = {};
    int next = 0;
};
H2dRing* g_h2d = new H2dRing;  // never freed (see above)

int h2d_ring_init(H2dRing& r)
{
    if (!r.pool) {
        const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
        auto* p = new CopyPool;
        p->workers = static_cast<int>(std::min(7u, std::max(1u, hw / 2)) - 1);
        for (int i = 0; i < p->workers; ++i) std::thread([p, i] { p->worker(i); }).detach();
        r.pool = p;
    }
    for (int k = 0; k < H2D_RING; ++k) {
        if (!r.chunk[k]) {
            void* ptr = nullptr;
            CR_HIP_RET(hipHostMalloc(&ptr, H2D_CHUNK, hipHostMallocDefault));
            r.chunk[k] = static_cast<char*>(ptr);
        }
        if (!r.ev[k]) CR_HIP_RET(hipEventCreateWithFlags(&r.ev[k], hipEventDisableTiming));
    }
    return CR_OK;
}
}  // namespace

int h2d_pageable(void* dst, const void* src, size_t bytes, hipStream_t s)
{
    if (bytes < H2D_DIRECT) {
        if (bytes) CR_HIP_RET(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s));
        return CR_OK;
    }
    H2dRing& r = *g_h2d;
    std::lock_guard<std::mutex> lk(r.mu);
    CR_RET(h2d_ring_init(r));
    for (size_t off = 0; off < bytes; off += H2D_CHUNK) {
        const int k = r.next;
        r.next = (r.next + 1) % H2D_RING;
        const size_t n = std::min(H2D_CHUNK, bytes - off);
        if (r.used[k]) CR_HIP_RET(hipEventSynchronize(r.ev[k]));  // its previous DMA has read it
        r.pool->copy(r.chunk[k], static_cast<const char*>(src) + off, n);
        CR_HIP_RET(hipMemcpyAsync(static_cast<char*>(dst) + off, r.chunk[k], n, hipMemcpyHostToDevice, s));
        CR_HIP_RET(hipEventRecord(r.ev[k], s));
        r.used[k] = true;
    }
    return CR_OK;
}

// Library-owned stream-ordered pool per device.  Its release threshold is
// "never", so memory returned by hipFreeAsync (scratch, freed results) stays
// mapped and the next allocation is a cache hit; the process's default pool is
// left untouched.  cr_mempool_trim() returns cached memory to the device.
static std::mutex g_pool_mu;
static hipMemPool_t g_pools[64] = {};

static hipMemPool_t library_pool()
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lock(g_pool_mu);
    if (!g_pools[dev]) {
        hipMemPoolProps props{};
        props.allocType = hipMemAllocationTypePinned;
        props.handleTypes = hipMemHandleTypeNone;
        props.location.type = hipMemLocationTypeDevice;
        props.location.id = dev;
        hipMemPool_t pool = nullptr;
        if (hipMemPoolCreate(&pool, &props) != hipSuccess) return nullptr;
        uint64_t never = ~0ull;
        (void)hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &never);
        g_pools[dev] = pool;
    }
    return g_pools[dev];
}

// Block cache in front of the pool: a block the library frees on a stream is
// kept and handed to the next allocation on that same stream that it fits
// (request <= size <= 2 x request), with no runtime call -- stream order makes
// the reuse safe.  Blocks of other streams stay until evicted (oldest first,
// beyond CACHE_MAX_BLOCKS or CACHE_MAX_BYTES) or until cr_mempool_trim().
struct CachedBlock {
    void* p;
    size_t bytes;
    int dev;
    hipStream_t stream;
};
static std::mutex g_cache_mu;
static std::vector<CachedBlock> g_cache;            // oldest first
static std::unordered_map<void*, std::pair<size_t, int>> g_live;  // size and device of blocks handed out
static size_t g_cache_bytes = 0;
constexpr size_t CACHE_MAX_BLOCKS = 32;
constexpr size_t CACHE_MAX_BYTES = size_t(16) << 30;

static void release_block(const CachedBlock& b)
{
    if (hipFreeAsync(b.p, b.stream) != hipSuccess) {  // e.g. the stream no longer exists
        (void)hipGetLastError();
        int cur = 0;
        (void)hipGetDevice(&cur);
        (void)hipSetDevice(b.dev);
        (void)hipDeviceSynchronize();
        (void)hipFree(b.p);
        (void)hipSetDevice(cur);
    }
}

// Test fault injection (cr_debug_fail_device_allocs): the allocations to let
// through, then the ones to fail.  Read under g_cache_mu.
static uint32_t g_fail_skip = 0, g_fail_count = 0;

int dev_alloc(void** p, size_t bytes, hipStream_t s)
{
    CR_HOST_PHASE("alloc");
    *p = nullptr;
    if (bytes == 0) bytes = 256;
    int dev = 0;
    CR_HIP_RET(hipGetDevice(&dev));
    {
        std::lock_guard<std::mutex> lock(g_cache_mu);
        if (g_fail_count) {
            if (g_fail_skip) {
                --g_fail_skip;
            } else {
                --g_fail_count;
                set_error("device allocation of %zu bytes failed (injected out-of-memory)", bytes);
                return CR_ERR_ALLOC;
            }
        }
        size_t best = g_cache.size();
        for (size_t i = 0; i < g_cache.size(); ++i) {
            const CachedBlock& b = g_cache[i];
            if (b.dev == dev && b.stream == s && b.bytes >= bytes && b.bytes <= 2 * bytes &&
                (best == g_cache.size() || b.bytes < g_cache[best].bytes))
                best = i;
        }
        if (best != g_cache.size()) {
            const CachedBlock b = g_cache[best];
            g_cache.erase(g_cache.begin() + static_cast<std::ptrdiff_t>(best));
            g_cache_bytes -= b.bytes;
            g_live[b.p] = {b.bytes, b.dev};
            *p = b.p;
            return CR_OK;
        }
    }
    hipMemPool_t pool = library_pool();
    hipError_t e = pool ? hipMallocFromPoolAsync(p, bytes, pool, s) : hipMallocAsync(p, bytes, s);
    if (e != hipSuccess) {
        set_error("hipMallocAsync(%zu bytes) failed: %s", bytes, hipGetErrorString(e));
        *p = nullptr;
        return e == hipErrorOutOfMemory ? CR_ERR_ALLOC : CR_ERR_HIP;
    }
    std::lock_guard<std::mutex> lock(g_cache_mu);
    g_live[*p] = {bytes, dev};
    return CR_OK;
}

int dev_free(void* p, hipStream_t s)
{
    if (!p) return CR_OK;
    CR_HOST_PHASE("free");
    std::vector<CachedBlock> evict;
    {
        std::lock_guard<std::mutex> lock(g_cache_mu);
        auto it = g_live.find(p);
        if (it == g_live.end()) {  // not a library block
            CR_HIP_RET(hipFreeAsync(p, s));
            return CR_OK;
        }
        g_cache.push_back({p, it->second.first, it->second.second, s});
        g_cache_bytes += it->second.first;
        g_live.erase(it);
        while (g_cache.size() > CACHE_MAX_BLOCKS || g_cache_bytes > CACHE_MAX_BYTES) {
            evict.push_back(g_cache.front());
            g_cache_bytes -= g_cache.front().bytes;
            g_cache.erase(g_cache.begin());
        }
    }
    for (const CachedBlock& b : evict) release_block(b);
    return CR_OK;
}

OutLayout plan_out(uint64_t n_meta, uint64_t kidx_len, uint64_t bmp_words, uint64_t arr_elems, uint64_t run_u16)
{
    Carver c;
    OutLayout L;
    L.bmp = c.add(bmp_words * 8);  // bitmap pool first: 256-byte aligned 8 KiB containers
    L.keys = c.add(n_meta * 2);
    L.types = c.add(n_meta);
    L.offsets = c.add(n_meta * 4);
    L.cards = c.add(n_meta * 2);
    L.kidx = c.add(kidx_len * 2);
    L.arr = c.add(arr_elems * 2);
    L.run = c.add(run_u16 * 2);
    L.total = c.total;
    return L;
}

int alloc_out(cr_gpu_roaring* out, const OutLayout& L, uint64_t n_meta, uint64_t kidx_len, uint64_t bmp_words,
              uint64_t arr_elems, uint64_t run_u16, hipStream_t s)
{
    void* base = nullptr;
    CR_RET(dev_alloc(&base, L.total, s));
    char* b = static_cast<char*>(base);
    out->_alloc_base = base;
    out->keys = n_meta ? reinterpret_cast<uint16_t*>(b + L.keys) : nullptr;
    out->types = n_meta ? reinterpret_cast<uint8_t*>(b + L.types) : nullptr;
    out->offsets = n_meta ? reinterpret_cast<uint32_t*>(b + L.offsets) : nullptr;
    out->cardinalities = n_meta ? reinterpret_cast<uint16_t*>(b + L.cards) : nullptr;
    out->key_index = kidx_len ? reinterpret_cast<uint16_t*>(b + L.kidx) : nullptr;
    out->bitmap_data = bmp_words ? reinterpret_cast<uint64_t*>(b + L.bmp) : nullptr;
    out->array_data = arr_elems ? reinterpret_cast<uint16_t*>(b + L.arr) : nullptr;
    out->run_data = run_u16 ? reinterpret_cast<uint16_t*>(b + L.run) : nullptr;
    return CR_OK;
}

void reset(cr_gpu_roaring* r) { std::memset(r, 0, sizeof(*r)); }

int free_async(cr_gpu_roaring* r, hipStream_t s)
{
    int rc = CR_OK;
    auto f = [&](void* p) {
        if (p && rc == CR_OK) rc = dev_free(p, s);
    };
    if (r->_alloc_base) {
        f(r->_alloc_base);
    } else {
        f(r->keys);
        f(r->types);
        f(r->offsets);
        f(r->cardinalities);
        f(r->bitmap_data);
        f(r->array_data);
        f(r->run_data);
        f(r->key_index);
    }
    reset(r);
    return rc;
}

__global__ void fill_u16_kernel(uint16_t* p, uint16_t v, uint64_t n)
{
    for (uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x)
        p[i] = v;
}

__global__ void fill_u32_kernel(uint32_t* p, uint32_t v, uint64_t n)
{
    for (uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x)
        p[i] = v;
}

static unsigned grid_for(uint64_t n, unsigned per_block, unsigned cap)
{
    uint64_t g = (n + per_block - 1) / per_block;
    if (g == 0) g = 1;
    return static_cast<unsigned>(g < cap ? g : cap);
}

int fill_u16(uint16_t* p, uint16_t v, uint64_t n, hipStream_t s)
{
    if (n == 0) return CR_OK;
    fill_u16_kernel<<<grid_for(n, 256, 4096), 256, 0, s>>>(p, v, n);
    CR_LAUNCH_CHECK();
    return CR_OK;
}

int fill_u32(uint32_t* p, uint32_t v, uint64_t n, hipStream_t s)
{
    if (n == 0) return CR_OK;
    fill_u32_kernel<<<grid_for(n, 256, 4096), 256, 0, s>>>(p, v, n);
    CR_LAUNCH_CHECK();
    return CR_OK;
}

bool g_timing_on = false;

struct TimingRec {
    std::string name;
    hipEvent_t start, stop;
    int dev;
};
static std::mutex g_timing_mu;
static std::vector<TimingRec> g_timing_recs;
// Events are recycled (creating one costs far more than recording it, and the
// timed calls should see as little of the timer as possible).  Each pool
// entry remembers the device it was created on.
static std::vector<std::pair<int, hipEvent_t>> g_event_pool;

static int current_device()
{
    int dev = 0;
    (void)hipGetDevice(&dev);
    return dev;
}

static hipEvent_t take_event()
{
    const int dev = current_device();
    {
        std::lock_guard<std::mutex> lock(g_timing_mu);
        for (size_t i = g_event_pool.size(); i-- > 0;) {
            if (g_event_pool[i].first == dev) {
                hipEvent_t e = g_event_pool[i].second;
                g_event_pool.erase(g_event_pool.begin() + static_cast<std::ptrdiff_t>(i));
                return e;
            }
        }
    }
    // Timing only: no system-scope fence (cache write-back) when the event is
    // recorded, which would otherwise slow the work that follows it.
    hipEvent_t e = nullptr;
    return hipEventCreateWithFlags(&e, hipEventDisableSystemFence) == hipSuccess ? e : nullptr;
}

static void give_event_locked(hipEvent_t e, int dev) { g_event_pool.emplace_back(dev, e); }


// Sampling: with period p, only every p-th launch of each kernel name is timed
// (the event markers add a few microseconds of queue time per launch).
static uint32_t g_timing_period = 1;
static std::unordered_map<const char*, uint64_t> g_timing_seen;

TimedLaunch::TimedLaunch(const char* n, hipStream_t s) : name(n), stream(s)
{
    if (!g_timing_on) return;
    {
        std::lock_guard<std::mutex> lock(g_timing_mu);
        if (g_timing_seen[n]++ % g_timing_period != 0) return;
    }
    start = take_event();
    if (start) (void)hipEventRecord(start, s);
}

TimedLaunch::~TimedLaunch()
{
    if (!start) return;
    hipEvent_t stop = take_event();
    const int dev = current_device();
    if (!stop) {
        std::lock_guard<std::mutex> lock(g_timing_mu);
        give_event_locked(start, dev);
        return;
    }
    (void)hipEventRecord(stop, stream);
    std::lock_guard<std::mutex> lock(g_timing_mu);
    g_timing_recs.push_back(TimingRec{name, start, stop, dev});
}

static std::vector<std::pair<std::string, double>> g_host_recs;

static double now_ms()
{
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

void record_host_ms(const char* name, double ms)
{
    std::lock_guard<std::mutex> lock(g_timing_mu);
    g_host_recs.emplace_back(std::string("host:") + name, ms);
}

HostPhase::HostPhase(const char* n) : name(n), t0(g_timing_on ? now_ms() : 0.0) {}

HostPhase::~HostPhase()
{
    if (g_timing_on) record_host_ms(name, now_ms() - t0);
}

uint32_t num_cus()
{
    static int cache[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cache[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
        cache[dev] = cus;
    }
    return static_cast<uint32_t>(cache[dev]);
}

uint64_t device_l2_bytes(int device)
{
    int dev = device;
    if (dev < 0 && hipGetDevice(&dev) != hipSuccess) dev = 0;
    int l2 = 0;
    if (hipDeviceGetAttribute(&l2, hipDeviceAttributeL2CacheSize, dev) != hipSuccess || l2 <= 0)
        l2 = 4 * 1024 * 1024;  // the reference's fallback (src/promote.cu:348-352)
    return static_cast<uint64_t>(l2);
}

// PROMOTE_AUTO, re-derived for gfx950 (the reference's rule is
// `2 * ceil(U/8) > L2`, src/promote.cu:334-367).  hipDeviceAttributeL2CacheSize
// reports one XCD's L2 (4 MiB); every XCD caches its own copy of what its waves
// read, and the 256 MB Infinity Cache behind them holds a whole 2^30 flat
// bitmap.  A sweep of the compressed (KEEP) and promoted (ALL) layouts over
// U = 2^20 .. 2^30 at 0.1 / 1 / 10% density (bench.py promote_sweep; the
// table is in profiles/promote_auto_sweep.md) found the promoted layout
// faster for uniform point queries by 1.8-5.4x at every universe where the
// layouts differ -- the lookup is one dependent load instead of a key index
// load plus a binary search, and both layouts stay cache-resident -- and its
// AND as fast (2^30, 0.1%) or up to 2.1x faster.  So on gfx950 promotion pays from the smallest
// universe swept, and the crossover moves down to where the reference's
// pinned verdicts allow: U = 10^6 must stay compressed
// (test/test_promote.cu:257-305), so promote once the flat bitmap exceeds
// 1/32 of one XCD's L2, i.e. 128 KiB (U > 2^20) on MI355X.  The rule sees only
// U; the memory term sits where the container count is known: upload() under
// AUTO keeps the layout when n_containers x 8 KiB x 2 >= ceil(U/8)
// (src/upload.cpp:106-118), so a sparse bitmap with a container at every key
// of 2^30 (2.3 MB at 0.1%) is not promoted to 134 MB there.
uint32_t resolve_auto_threshold(uint32_t universe_size, int device)
{
    if (universe_size == 0) return CR_PROMOTE_KEEP_DEFAULT;
    const uint64_t flat = (static_cast<uint64_t>(universe_size) + 7u) / 8u;
    return flat * 32u > device_l2_bytes(device) ? CR_PROMOTE_ALL : CR_PROMOTE_KEEP_DEFAULT;
}

}  // namespace crimpl

using namespace crimpl;

extern "C" {

const char* cr_last_error(void) { return g_last_error.c_str(); }

int cr_free(cr_gpu_roaring* bm)
{
    if (!bm) return CR_OK;
    int rc = free_async(bm, nullptr);
    if (rc == CR_OK) CR_HIP_RET(hipStreamSynchronize(nullptr));
    return rc;
}

int cr_free_async(cr_gpu_roaring* bm, cr_stream_t stream)
{
    if (!bm) return CR_OK;
    return free_async(bm, as_stream(stream));
}

int cr_resolve_auto_threshold(uint32_t universe_size, int device_id, uint32_t* out_threshold)
{
    if (!out_threshold) {
        set_error("cr_resolve_auto_threshold: null output");
        return CR_ERR_INVALID;
    }
    *out_threshold = resolve_auto_threshold(universe_size, device_id);
    return CR_OK;
}

int cr_device_l2_bytes(int device_id, uint64_t* out_bytes)
{
    if (!out_bytes) return CR_ERR_INVALID;
    *out_bytes = device_l2_bytes(device_id);
    return CR_OK;
}

int cr_make_view(const cr_gpu_roaring* b, cr_gpu_roaring_view* v)
{
    if (!b || !v) {
        set_error("cr_make_view: null argument");
        return CR_ERR_INVALID;
    }
    v->keys = b->keys;
    v->types = b->types;
    v->offsets = b->offsets;
    v->cardinalities = b->cardinalities;
    v->n_containers = b->n_containers;
    v->bitmap_data = b->bitmap_data;
    v->array_data = b->array_data;
    v->run_data = b->run_data;
    v->key_index = b->key_index;
    v->max_key = b->max_key;
    v->all_bitmap = b->n_array_containers == 0 && b->n_run_containers == 0 && b->key_index != nullptr;
    v->negated = b->negated;
    return CR_OK;
}

int cr_device_malloc(void** ptr, size_t bytes)
{
    CR_HIP_RET(hipMalloc(ptr, bytes ? bytes : 1));
    return CR_OK;
}

int cr_device_free(void* ptr)
{
    CR_HIP_RET(hipFree(ptr));
    return CR_OK;
}

int cr_memcpy_h2d(void* dst, const void* src, size_t bytes)
{
    if (bytes) CR_HIP_RET(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return CR_OK;
}

int cr_memcpy_d2h(void* dst, const void* src, size_t bytes)
{
    if (bytes) CR_HIP_RET(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return CR_OK;
}

int cr_stream_synchronize(cr_stream_t stream)
{
    CR_HIP_RET(hipStreamSynchronize(as_stream(stream)));
    return CR_OK;
}

int cr_mempool_trim(int device_id, size_t keep_bytes)
{
    int dev = device_id;
    if (dev < 0) CR_HIP_RET(hipGetDevice(&dev));
    if (dev >= 64) return CR_ERR_INVALID;
    std::vector<CachedBlock> drop;
    {
        std::lock_guard<std::mutex> lock(g_cache_mu);
        for (size_t i = 0; i < g_cache.size();) {
            if (g_cache[i].dev == dev) {
                drop.push_back(g_cache[i]);
                g_cache_bytes -= g_cache[i].bytes;
                g_cache.erase(g_cache.begin() + static_cast<std::ptrdiff_t>(i));
            } else {
                ++i;
            }
        }
    }
    for (const CachedBlock& b : drop) release_block(b);
    std::lock_guard<std::mutex> lock(g_pool_mu);
    if (g_pools[dev]) {
        CR_HIP_RET(hipDeviceSynchronize());
        CR_HIP_RET(hipMemPoolTrimTo(g_pools[dev], keep_bytes));
    }
    return CR_OK;
}

int cr_debug_fail_device_allocs(uint32_t skip, uint32_t count)
{
    std::lock_guard<std::mutex> lock(g_cache_mu);
    g_fail_skip = count ? skip : 0u;
    g_fail_count = count;
    return CR_OK;
}

int cr_timing_enable(int on)
{
    std::lock_guard<std::mutex> lock(g_timing_mu);
    for (auto& r : g_timing_recs) {
        (void)hipEventSynchronize(r.stop);  // recorded work must pass the events before they are reused
        give_event_locked(r.start, r.dev);
        give_event_locked(r.stop, r.dev);
    }
    g_timing_recs.clear();
    g_host_recs.clear();
    g_timing_seen.clear();
    g_timing_on = on != 0;
    g_timing_period = on > 1 ? static_cast<uint32_t>(on) : 1u;
    return CR_OK;
}

int cr_timing_report(char* buf, size_t cap)
{
    if (!buf || cap == 0) return CR_ERR_INVALID;
    std::lock_guard<std::mutex> lock(g_timing_mu);
    // name -> every timed launch's ms, in first-seen order
    std::vector<std::pair<std::string, std::vector<double>>> agg;
    auto slot = [&](const std::string& name) -> std::vector<double>& {
        auto it = std::find_if(agg.begin(), agg.end(), [&](auto& a) { return a.first == name; });
        if (it != agg.end()) return it->second;
        agg.push_back({name, {}});
        return agg.back().second;
    };
    for (auto& r : g_timing_recs) {
        CR_HIP_RET(hipEventSynchronize(r.stop));
        float ms = 0.f;
        CR_HIP_RET(hipEventElapsedTime(&ms, r.start, r.stop));
        slot(r.name).push_back(ms);
    }
    for (auto& h : g_host_recs) slot(h.first).push_back(h.second);
    // one line per name: launches, total ms, median ms (the upper median for an
    // even count, so a single outlier launch cannot move it)
    std::string out;
    char line[256];
    for (auto& a : agg) {
        std::vector<double> v = a.second;
        double total = 0.0;
        for (double x : v) total += x;
        std::sort(v.begin(), v.end());
        snprintf(line, sizeof(line), "%s %llu %.6f %.6f\n", a.first.c_str(), static_cast<unsigned long long>(v.size()),
                 total, v[v.size() / 2]);
        out += line;
    }
    snprintf(buf, cap, "%s", out.c_str());
    return CR_OK;
}

}  // extern "C"

// End-to-end check of the C++ drop-in surface (namespaces cu_roaring and
// cu_roaring::v2) as a reference user would call it, including the
// header-only device queries from a kernel of the caller's own.  Each result
// is checked against a host truth built here from the input ids.  Prints
// "api_check: OK" and exits 0 when every check passes.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <set>
#include <stdexcept>
#include <string>
#include <vector>

#include <cu_roaring/cu_roaring.cuh>
#include <cu_roaring/device/roaring_view.cuh>
#include <cu_roaring/device/roaring_warp_query.cuh>
#include <cu_roaring_v2/api.hpp>
#include <cu_roaring_v2/query.cuh>

#define HIP_OK(x)                                                                      \
    do {                                                                               \
        hipError_t e_ = (x);                                                           \
        if (e_ != hipSuccess) {                                                        \
            std::fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_)); \
            std::exit(2);                                                              \
        }                                                                              \
    } while (0)

static int g_fail = 0;
#define CHECK(c)                                                              \
    do {                                                                      \
        if (!(c)) {                                                           \
            std::fprintf(stderr, "CHECK failed %s:%d: %s\n", __FILE__, __LINE__, #c); \
            ++g_fail;                                                         \
        }                                                                     \
    } while (0)

// A caller's kernel: both v1 device queries on one view.
__global__ void user_query_v1(cu_roaring::GpuRoaringView v, const uint32_t* ids, uint32_t n, uint8_t* a, uint8_t* b)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    const bool in = i < n;
    const uint32_t id = in ? ids[i] : 0u;
    const bool w = cu_roaring::warp_contains(v, id);  // every lane of the wavefront takes part
    if (in) {
        a[i] = v.contains(id) ? 1 : 0;
        b[i] = w ? 1 : 0;
    }
}

// A caller's kernel over the batch: bitmap per query, and one view.
__global__ void user_query_v2(cu_roaring::v2::GpuRoaringBatch batch, cu_roaring::v2::GpuRoaringView view,
                              const uint32_t* ids, const uint32_t* which, uint32_t n, uint8_t* a, uint8_t* b)
{
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    a[i] = cu_roaring::v2::contains(batch, which[i], ids[i]) ? 1 : 0;
    b[i] = cu_roaring::v2::contains(view, ids[i]) ? 1 : 0;
}

static std::vector<uint8_t> d2h_u8(const uint8_t* d, size_t n)
{
    std::vector<uint8_t> h(n);
    HIP_OK(hipMemcpy(h.data(), d, n, hipMemcpyDeviceToHost));
    return h;
}

static std::vector<cu_roaring::HostContainer> containers_of(const std::vector<uint32_t>& sorted_ids,
                                                            std::vector<std::vector<uint16_t>>& store)
{
    // array containers (<= 4096 values) or bitsets, like CRoaring without runs
    std::vector<cu_roaring::HostContainer> out;
    size_t i = 0;
    while (i < sorted_ids.size()) {
        const uint32_t key = sorted_ids[i] >> 16;
        size_t j = i;
        while (j < sorted_ids.size() && (sorted_ids[j] >> 16) == key) ++j;
        const size_t card = j - i;
        cu_roaring::HostContainer c{};
        c.key = static_cast<uint16_t>(key);
        c.cardinality = static_cast<int32_t>(card);
        if (card <= 4096) {
            store.emplace_back();
            for (size_t k = i; k < j; ++k) store.back().push_back(static_cast<uint16_t>(sorted_ids[k] & 0xFFFFu));
            c.typecode = CR_TC_ARRAY;
        } else {
            store.emplace_back(4096, 0);  // 1024 u64 as 4096 u16
            auto* w = reinterpret_cast<uint64_t*>(store.back().data());
            for (size_t k = i; k < j; ++k) w[(sorted_ids[k] & 0xFFFFu) >> 6] |= 1ull << (sorted_ids[k] & 63u);
            c.typecode = CR_TC_BITSET;
        }
        out.push_back(c);
        i = j;
    }
    for (size_t k = 0; k < out.size(); ++k) out[k].data = store[k].data();
    return out;
}

int main()
{
    namespace cr = cu_roaring;
    std::mt19937 gen(7);
    const uint32_t U = 1u << 22;
    std::vector<uint32_t> a_ids(300000), b_ids(80000);
    for (auto& x : a_ids) x = gen() % U;
    for (auto& x : b_ids) x = gen() % U;
    std::set<uint32_t> sa(a_ids.begin(), a_ids.end()), sb(b_ids.begin(), b_ids.end());

    // ---- v1: upload, set operation, multi_and -------------------------------------
    cr::GpuRoaring A = cr::upload_from_ids(a_ids.data(), static_cast<uint32_t>(a_ids.size()), U);
    cr::GpuRoaring B = cr::upload_from_ids(b_ids.data(), static_cast<uint32_t>(b_ids.size()), U);
    CHECK(A.total_cardinality == sa.size() && B.total_cardinality == sb.size());
    cr::GpuRoaring AB = cr::set_operation(A, B, cr::SetOp::AND);
    const cr::GpuRoaring both[2] = {A, B};
    cr::GpuRoaring M = cr::multi_and(both, 2);
    std::vector<uint32_t> inter;
    std::set_intersection(sa.begin(), sa.end(), sb.begin(), sb.end(), std::back_inserter(inter));

    // ---- device queries from the caller's kernel ---------------------------------------
    const uint32_t nq = 100000;
    std::vector<uint32_t> q(nq);
    for (auto& x : q) x = gen() % (U + 4096);
    uint32_t* dq;
    uint8_t *d1, *d2;
    HIP_OK(hipMalloc(&dq, nq * 4));
    HIP_OK(hipMalloc(&d1, nq));
    HIP_OK(hipMalloc(&d2, nq));
    HIP_OK(hipMemcpy(dq, q.data(), nq * 4, hipMemcpyHostToDevice));
    for (const cr::GpuRoaring* g : {&A, &M}) {
        user_query_v1<<<(nq + 255) / 256, 256>>>(cr::make_view(*g), dq, nq, d1, d2);
        HIP_OK(hipDeviceSynchronize());
        auto r1 = d2h_u8(d1, nq), r2 = d2h_u8(d2, nq);
        std::set<uint32_t> truth = g == &A ? sa : std::set<uint32_t>(inter.begin(), inter.end());
        bool ok = true;
        for (uint32_t i = 0; i < nq; ++i) {
            const uint8_t t = truth.count(q[i]) ? 1 : 0;
            ok &= r1[i] == t && r2[i] == t;
        }
        CHECK(ok);
    }

    // ---- conversions ---------------------------------------------------------------------
    uint32_t* bits = cr::decompress_to_bitset(AB);
    std::vector<uint32_t> hb((U + 31) / 32);
    HIP_OK(hipMemcpy(hb.data(), bits, hb.size() * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipFree(bits));
    {
        bool ok = true;
        size_t pc = 0;
        for (uint32_t w : hb) pc += __builtin_popcount(w);
        ok &= pc == inter.size();
        for (uint32_t x : inter) ok &= ((hb[x >> 5] >> (x & 31)) & 1u) != 0;
        CHECK(ok);
    }
    int64_t* ids_out = cr::enumerate_ids(A);
    std::vector<int64_t> he(sa.size());
    HIP_OK(hipDeviceSynchronize());
    HIP_OK(hipMemcpy(he.data(), ids_out, he.size() * 8, hipMemcpyDeviceToHost));
    HIP_OK(hipFree(ids_out));
    CHECK(std::equal(he.begin(), he.end(), sa.begin(), [](int64_t x, uint32_t y) { return x == static_cast<int64_t>(y); }));
    cr::GpuRoaring P = cr::promote_to_bitmap(A);
    cr::GpuRoaring D = cr::gpu_roaring_deep_copy(A);
    HIP_OK(hipDeviceSynchronize());
    CHECK(P.n_bitmap_containers == P.n_containers && D.total_cardinality == A.total_cardinality);

    // ---- portable format round trip ------------------------------------------------------
    std::vector<uint8_t> bytes = cr::portable_serialize(A);
    CHECK(bytes.size() == cr::portable_size_in_bytes(A));
    cr::GpuRoaring R = cr::portable_deserialize(bytes.data(), bytes.size(), U);
    CHECK(R.total_cardinality == sa.size() && cr::portable_serialize(R) == bytes);

    // ---- v2 batch --------------------------------------------------------------------------
    namespace v2 = cu_roaring::v2;
    std::vector<std::vector<uint32_t>> sets(4);
    std::vector<std::vector<std::vector<uint16_t>>> stores(4);
    std::vector<std::vector<cr::HostContainer>> lists(4);
    for (int b = 0; b < 4; ++b) {
        std::set<uint32_t> s;
        for (int k = 0; k < 60000; ++k) s.insert(gen() % (1u << 20));
        for (uint32_t x = 0; x < 20000; ++x) s.insert(x);  // shared ids: a non-empty intersection
        sets[b].assign(s.begin(), s.end());
        lists[b] = containers_of(sets[b], stores[b]);
    }
    const cr::HostContainer* ptrs[4] = {lists[0].data(), lists[1].data(), lists[2].data(), lists[3].data()};
    const uint32_t counts[4] = {static_cast<uint32_t>(lists[0].size()), static_cast<uint32_t>(lists[1].size()),
                                static_cast<uint32_t>(lists[2].size()), static_cast<uint32_t>(lists[3].size())};
    v2::GpuRoaringBatch batch = v2::upload_batch(ptrs, counts, 4);
    for (int b = 0; b < 4; ++b) CHECK(batch.host_total_cardinalities[b] == sets[b].size());
    v2::GpuRoaringBatch pb = v2::promote_batch(batch);
    const uint32_t idx[3] = {0, 1, 3};
    v2::GpuRoaringBatch anded = v2::multi_and(pb, idx, 3);
    std::vector<uint32_t> i01, i013;
    std::set_intersection(sets[0].begin(), sets[0].end(), sets[1].begin(), sets[1].end(), std::back_inserter(i01));
    std::set_intersection(i01.begin(), i01.end(), sets[3].begin(), sets[3].end(), std::back_inserter(i013));
    CHECK(anded.host_total_cardinalities[0] == i013.size());
    bool threw = false;
    try {
        v2::multi_and(batch, idx, 3);  // array containers: promote first
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    CHECK(threw);
    threw = false;
    try {
        v2::make_view(batch, 4);
    } catch (const std::out_of_range&) {
        threw = true;
    }
    CHECK(threw);
    std::vector<uint32_t> which(nq);
    for (uint32_t i = 0; i < nq; ++i) {
        which[i] = gen() % 4;
        q[i] = gen() % (1u << 20);
    }
    uint32_t* dw;
    HIP_OK(hipMalloc(&dw, nq * 4));
    HIP_OK(hipMemcpy(dw, which.data(), nq * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dq, q.data(), nq * 4, hipMemcpyHostToDevice));
    user_query_v2<<<(nq + 255) / 256, 256>>>(batch, v2::make_view(anded, 0), dq, dw, nq, d1, d2);
    HIP_OK(hipDeviceSynchronize());
    {
        auto r1 = d2h_u8(d1, nq), r2 = d2h_u8(d2, nq);
        bool ok = true;
        for (uint32_t i = 0; i < nq; ++i) {
            const auto& s = sets[which[i]];
            ok &= r1[i] == (std::binary_search(s.begin(), s.end(), q[i]) ? 1 : 0);
            ok &= r2[i] == (std::binary_search(i013.begin(), i013.end(), q[i]) ? 1 : 0);
        }
        CHECK(ok);
    }
    v2::free_batch(anded);
    v2::free_batch(pb);
    v2::free_batch(batch);

    // ---- an allocation failure surfaces as std::runtime_error -------------------------
    // (the reference's CUDA_CHECK contract, include/cu_roaring/detail/utils.cuh:9-18):
    // the first, then the third device allocation of each call fails.
    for (uint32_t skip : {0u, 2u}) {
        int caught = 0;
        cr_debug_fail_device_allocs(skip, 1);
        try {
            cr::GpuRoaring X = cr::upload_from_ids(a_ids.data(), static_cast<uint32_t>(a_ids.size()), U);
            cr::gpu_roaring_free(X);
        } catch (const std::runtime_error& e) {
            caught = std::string(e.what()).find("out-of-memory") != std::string::npos ? 1 : 2;
        }
        cr_debug_fail_device_allocs(0, 1);
        try {
            cr::GpuRoaring X = cr::set_operation(A, B, cr::SetOp::OR);
            cr::gpu_roaring_free(X);
        } catch (const std::runtime_error& e) {
            caught += std::string(e.what()).find("out-of-memory") != std::string::npos ? 10 : 20;
        }
        cr_debug_fail_device_allocs(0, 0);
        CHECK(caught == 11 || (skip == 2 && caught == 10));  // an upload may make fewer than 3 allocations
    }
    {  // and the library still works afterwards
        cr::GpuRoaring X = cr::upload_from_ids(a_ids.data(), static_cast<uint32_t>(a_ids.size()), U);
        CHECK(X.total_cardinality == sa.size());
        cr::gpu_roaring_free(X);
    }
    for (cr::GpuRoaring* g : {&A, &B, &AB, &M, &P, &D, &R}) cr::gpu_roaring_free(*g);
    HIP_OK(hipFree(dq));
    HIP_OK(hipFree(dw));
    HIP_OK(hipFree(d1));
    HIP_OK(hipFree(d2));
    if (g_fail) {
        std::printf("api_check: %d check(s) failed\n", g_fail);
        return 1;
    }
    std::printf("api_check: OK\n");
    return 0;
}

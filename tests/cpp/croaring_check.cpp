// The reference's roaring_bitmap_t* entry points, compiled with
// CU_ROARING_WITH_CROARING against the test-only CRoaring stand-in in
// croaring_shim/ (CRoaring's public struct layout, backed by roaring-lite):
//   upload(bm, stream, thr), upload(bm, U, stream, thr), get_meta(bm)
//     (include/cu_roaring/detail/upload.cuh:19-41 in the reference), and
//   v2::upload_batch(roaring_bitmap_t* const*, n, stream)
//     (v2/include/cu_roaring_v2/api.hpp:22-24).
// Each is checked byte for byte against the HostContainer path (a container
// list built here straight from roaring-lite, not through the adapter), and
// each upload's logical set against a flat bitset of its input ids.  The
// complement of upload(bm, U) goes through roaring_bitmap_flip_inplace on one
// side and the library's host complement on the other.
// Prints "croaring_check: OK" and exits 0 when every check passes.
#define CU_ROARING_WITH_CROARING 1
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include <cu_roaring/cu_roaring.cuh>
#include <cu_roaring_v2/api.hpp>

#include "oracle.h"

#define HIP_OK(x)                                                                          \
    do {                                                                                   \
        hipError_t e_ = (x);                                                               \
        if (e_ != hipSuccess) {                                                            \
            std::fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_)); \
            std::exit(2);                                                                  \
        }                                                                                  \
    } while (0)

static int g_fail = 0;
static std::string g_case;
#define CHECK(c)                                                                                          \
    do {                                                                                                  \
        if (!(c)) {                                                                                       \
            std::fprintf(stderr, "CHECK failed [%s] %s:%d: %s\n", g_case.c_str(), __FILE__, __LINE__, #c); \
            ++g_fail;                                                                                     \
        }                                                                                                 \
    } while (0)

namespace cr = cu_roaring;

template <class T>
static std::vector<T> d2h(const T* d, size_t n)
{
    std::vector<T> h(n);
    if (n) HIP_OK(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
    return h;
}

// Everything a GpuRoaring holds, in host memory (pools in full).
struct Dump {
    std::vector<uint16_t> keys, cards, key_index, arrays, runs;
    std::vector<uint8_t> types;
    std::vector<uint32_t> offsets;
    std::vector<uint64_t> bitmaps;
    uint32_t n_c, n_b, n_a, n_r, U, max_key, apb, rpb;
    uint64_t total;
    bool negated;
    bool operator==(const Dump& o) const
    {
        return keys == o.keys && cards == o.cards && key_index == o.key_index && arrays == o.arrays &&
               runs == o.runs && types == o.types && offsets == o.offsets && bitmaps == o.bitmaps && n_c == o.n_c &&
               n_b == o.n_b && n_a == o.n_a && n_r == o.n_r && U == o.U && max_key == o.max_key && apb == o.apb &&
               rpb == o.rpb && total == o.total && negated == o.negated;
    }
};

static Dump dump(const cr::GpuRoaring& g)
{
    Dump d;
    d.n_c = g.n_containers;
    d.n_b = g.n_bitmap_containers;
    d.n_a = g.n_array_containers;
    d.n_r = g.n_run_containers;
    d.U = g.universe_size;
    d.max_key = g.max_key;
    d.apb = g.array_pool_bytes;
    d.rpb = g.run_pool_bytes;
    d.total = g.total_cardinality;
    d.negated = g.negated;
    d.keys = d2h(g.keys, g.n_containers);
    d.cards = d2h(g.cardinalities, g.n_containers);
    d.offsets = d2h(g.offsets, g.n_containers);
    d.types = d2h(reinterpret_cast<const uint8_t*>(g.types), g.n_containers);
    d.key_index = g.key_index ? d2h(g.key_index, g.max_key + 1ull) : std::vector<uint16_t>{};
    d.bitmaps = d2h(g.bitmap_data, g.n_bitmap_containers * 1024ull);
    d.arrays = d2h(g.array_data, g.array_pool_bytes / 2u);
    d.runs = d2h(g.run_data, g.run_pool_bytes / 2u);
    return d;
}

// The HostContainer list of the same bitmap, straight from roaring-lite.
struct Lite {
    rl_bitmap* b;
    std::vector<cr::HostContainer> hc;
    Lite(const std::vector<uint32_t>& ids, bool run_opt) : b(rl_from_ids(ids.data(), ids.size()))
    {
        if (run_opt) rl_run_optimize(b);
        hc.resize(rl_n_containers(b));
        for (uint32_t i = 0; i < hc.size(); ++i) {
            uint16_t key;
            uint8_t tc;
            int32_t card;
            const void* data;
            rl_container_info(b, i, &key, &tc, &card, &data);
            hc[i].key = key;
            hc[i].typecode = tc;
            hc[i].cardinality = card;
            hc[i].data = data;
        }
    }
    ~Lite() { rl_destroy(b); }
    uint32_t n() const { return static_cast<uint32_t>(hc.size()); }
};

// The logical set of `g` (decompressed, complement applied) equals `ids` below U.
static bool logical_matches(const cr::GpuRoaring& g, const std::vector<uint32_t>& ids, uint32_t U)
{
    if (U == 0) return true;
    uint32_t* bits = cr::decompress_to_bitset(g);
    HIP_OK(hipDeviceSynchronize());
    const uint32_t n_words = (U + 31u) / 32u;
    std::vector<uint32_t> got = d2h(bits, n_words);
    HIP_OK(hipFree(bits));
    std::vector<uint32_t> want(n_words, 0);
    for (uint32_t x : ids)
        if (x < U) want[x >> 5] |= 1u << (x & 31u);
    return got == want;
}

static void check_case(const char* name, const std::vector<uint32_t>& ids, bool run_opt, uint32_t U)
{
    g_case = name;
    std::printf("CASE %s: %zu ids, run_optimize %d, U %u\n", name, ids.size(), run_opt ? 1 : 0, U);
    std::fflush(stdout);
    Lite lite(ids, run_opt);
    roaring_bitmap_t* bm = shim_bitmap_of_ids(ids.data(), ids.size(), run_opt);
    CHECK(roaring_bitmap_get_cardinality(bm) == rl_cardinality(lite.b));

    // get_meta(bm) -- src/upload.cpp:31-71
    const cr::GpuRoaringMeta m1 = cr::get_meta(bm);
    const cr::GpuRoaringMeta m2 = cr::get_meta(lite.hc.data(), lite.n());
    CHECK(std::memcmp(&m1, &m2, sizeof(m1)) == 0);

    for (uint32_t thr : {cr::PROMOTE_AUTO, cr::PROMOTE_KEEP_DEFAULT, cr::PROMOTE_ALL, 100u}) {
        // upload(bm, stream, thr): universe from the last key, no complement
        cr::GpuRoaring a = cr::upload(bm, 0, thr);
        cr::GpuRoaring b = cr::upload(lite.hc.data(), lite.n(), 0, thr);
        CHECK(dump(a) == dump(b));
        CHECK(logical_matches(a, ids, a.universe_size));
        cr::gpu_roaring_free(a);
        cr::gpu_roaring_free(b);
        // upload(bm, U, stream, thr): complement when card > U/2
        cr::GpuRoaring c = cr::upload(bm, U, 0, thr);
        cr::GpuRoaring d = cr::upload(lite.hc.data(), lite.n(), U, 0, thr);
        const Dump dc = dump(c);
        CHECK(dc == dump(d));
        CHECK(c.total_cardinality == rl_cardinality(lite.b));  // the logical count (src/upload.cpp:306-307)
        CHECK(c.negated == (rl_cardinality(lite.b) > U / 2u));
        CHECK(logical_matches(c, ids, U));
        cr::gpu_roaring_free(c);
        cr::gpu_roaring_free(d);
    }
    roaring_bitmap_free(bm);
}

int main()
{
    std::mt19937 gen(11);
    const uint32_t U = 1u << 22;
    std::vector<uint32_t> sparse(20000), dense, runs, mixed;
    for (auto& x : sparse) x = gen() % U;
    for (uint32_t x = 0; x < U; ++x)
        if (gen() % 100 < 70) dense.push_back(x);  // 70%: complement with U
    for (uint32_t r = 0; r < 200; ++r) {
        const uint32_t st = gen() % (U - 70000), ln = 1000 + gen() % 64000;
        for (uint32_t x = st; x < st + ln; ++x) runs.push_back(x);
    }
    for (uint32_t key = 0; key < 48; ++key) {  // arrays, bitsets, runs and one full container
        const uint32_t base = key << 16;
        if (key % 4 == 0) {
            for (uint32_t x = 0; x < 300; ++x) mixed.push_back(base + gen() % 65536);
        } else if (key % 4 == 1) {
            for (uint32_t x = 0; x < 30000; ++x) mixed.push_back(base + gen() % 65536);
        } else if (key % 4 == 2) {
            for (uint32_t x = 5; x < 40000; ++x) mixed.push_back(base + x);
        } else if (key == 7) {
            for (uint32_t x = 0; x < 65536; ++x) mixed.push_back(base + x);
        }
    }
    check_case("sparse arrays", sparse, false, U);
    check_case("dense (complement)", dense, false, U);
    check_case("dense run-optimized (complement)", dense, true, U);
    check_case("runs", runs, true, U);
    check_case("mixed", mixed, true, U);
    check_case("mixed, odd U", mixed, true, (48u << 16) + 11u);
    check_case("single id", std::vector<uint32_t>{123457}, false, U);

    // v2::upload_batch(roaring_bitmap_t* const*, n, stream)
    {
        g_case = "upload_batch";
        std::printf("CASE v2 upload_batch\n");
        std::fflush(stdout);
        namespace v2 = cu_roaring::v2;
        const std::vector<uint32_t>* sets[4] = {&sparse, &runs, &mixed, &dense};
        std::vector<Lite*> lites;
        std::vector<roaring_bitmap_t*> bms;
        std::vector<const cr::HostContainer*> ptrs;
        std::vector<uint32_t> counts;
        for (int b = 0; b < 4; ++b) {
            lites.push_back(new Lite(*sets[b], b != 0));
            bms.push_back(shim_bitmap_of_ids(sets[b]->data(), sets[b]->size(), b != 0));
            ptrs.push_back(lites.back()->hc.data());
            counts.push_back(lites.back()->n());
        }
        v2::GpuRoaringBatch x = v2::upload_batch(bms.data(), 4);
        v2::GpuRoaringBatch y = v2::upload_batch(ptrs.data(), counts.data(), 4);
        CHECK(x.n_bitmaps == y.n_bitmaps && x.total_containers == y.total_containers &&
              x.n_bitmap_containers_total == y.n_bitmap_containers_total &&
              x.array_pool_bytes == y.array_pool_bytes && x.run_pool_bytes == y.run_pool_bytes);
        const uint32_t n_c = y.total_containers;
        const uint32_t n_ki = y.host_key_index_starts[4];
        CHECK(d2h(x.keys, n_c) == d2h(y.keys, n_c));
        CHECK(d2h(reinterpret_cast<const uint8_t*>(x.types), n_c) == d2h(reinterpret_cast<const uint8_t*>(y.types), n_c));
        CHECK(d2h(x.offsets, n_c) == d2h(y.offsets, n_c));
        CHECK(d2h(x.cardinalities, n_c) == d2h(y.cardinalities, n_c));
        CHECK(d2h(x.key_indices, n_ki) == d2h(y.key_indices, n_ki));
        CHECK(d2h(x.bitmap_data, y.n_bitmap_containers_total * 1024ull) ==
              d2h(y.bitmap_data, y.n_bitmap_containers_total * 1024ull));
        CHECK(d2h(x.array_data, y.array_pool_bytes / 2u) == d2h(y.array_data, y.array_pool_bytes / 2u));
        CHECK(d2h(x.run_data, y.run_pool_bytes / 2u) == d2h(y.run_data, y.run_pool_bytes / 2u));
        for (int b = 0; b < 4; ++b) {
            CHECK(x.host_total_cardinalities[b] == rl_cardinality(lites[b]->b));
            CHECK(x.host_total_cardinalities[b] == y.host_total_cardinalities[b]);
            CHECK(x.host_universe_sizes[b] == y.host_universe_sizes[b]);
            CHECK(x.host_container_starts[b + 1] == y.host_container_starts[b + 1]);
            CHECK(x.host_n_bitmap_containers[b] == y.host_n_bitmap_containers[b]);
        }
        v2::free_batch(x);
        v2::free_batch(y);
        for (int b = 0; b < 4; ++b) {
            roaring_bitmap_free(bms[b]);
            delete lites[b];
        }
    }
    if (g_fail) {
        std::printf("croaring_check: %d check(s) failed\n", g_fail);
        return 1;
    }
    std::printf("croaring_check: OK\n");
    return 0;
}

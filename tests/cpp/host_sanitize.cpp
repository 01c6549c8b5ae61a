// The library's host-side C++ (cu-roaring-bitmap_amd/host/api.cpp: the Roaring
// portable-format parser, the host complement of upload(bm, U), the C++
// wrappers) compiled with g++ and AddressSanitizer + UndefinedBehaviorSanitizer,
// without a GPU.  The device entry points api.cpp calls are replaced here by
// stubs; cr_upload_containers records the containers it is handed, which this
// program decodes (every payload byte is read, so a container that points
// outside its input shows up as an ASan report).
//
//   host_sanitize DIR   reads DIR/case_<i>.bin (portable bytes, written by
//                       roaring-lite) and DIR/case_<i>.ids (the set: u32
//                       universe, then the sorted u32 ids) for i = 0, 1, ...
//
// For each case: the parse gives exactly the set; with the universe given and
// more than half of it set, the complement is handed over, and it is the
// complement within [0, U); then 3000 mutated copies (byte flips, cuts,
// extensions) are parsed, each rejected with CR_ERR_INVALID or handed over as
// containers that lie inside the input.  Prints "host_sanitize: OK" when every check passes.
#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <random>
#include <string>
#include <vector>

#include "cu_roaring_abi.h"

namespace crimpl {
void set_error(const char*, ...) {}
}  // namespace crimpl

extern "C" {
const char* cr_last_error(void) { return "stub"; }

static std::vector<uint32_t> g_ids;  // the set the last cr_upload_containers call was handed
static uint32_t g_universe = 0;
static bool g_complemented = false;
static int g_uploads = 0;
static int g_fail = 0;

#define CHECK(c)                                                              \
    do {                                                                      \
        if (!(c)) {                                                           \
            std::printf("CHECK failed %s:%d: %s\n", __FILE__, __LINE__, #c);  \
            ++g_fail;                                                         \
        }                                                                     \
    } while (0)

int cr_upload_containers(const cr_host_container* c, uint32_t n, uint32_t universe_size, bool complemented,
                         uint64_t, cr_stream_t, uint32_t, cr_gpu_roaring* out)
{
    ++g_uploads;
    g_ids.clear();
    g_universe = universe_size;
    g_complemented = complemented;
    for (uint32_t i = 0; i < n; ++i) {
        if (i > 0 && c[i - 1].key >= c[i].key) return CR_ERR_INVALID;  // as the library checks
        const uint32_t base = static_cast<uint32_t>(c[i].key) << 16;
        const int32_t card = c[i].cardinality;
        if (card < 0 || (card > 0 && !c[i].data)) return CR_ERR_INVALID;
        if (c[i].typecode == CR_TC_BITSET) {
            uint64_t w[1024];
            std::memcpy(w, c[i].data, sizeof(w));  // reads all 8 KiB (may be unaligned)
            for (uint32_t k = 0; k < 1024u; ++k)
                for (uint64_t x = w[k]; x; x &= x - 1) g_ids.push_back(base + k * 64u + __builtin_ctzll(x));
        } else if (c[i].typecode == CR_TC_ARRAY) {
            std::vector<uint16_t> a(static_cast<size_t>(card));
            if (card) std::memcpy(a.data(), c[i].data, a.size() * 2);
            for (uint16_t v : a) g_ids.push_back(base + v);
        } else if (c[i].typecode == CR_TC_RUN) {
            std::vector<uint16_t> r(2 * static_cast<size_t>(card));
            if (card) std::memcpy(r.data(), c[i].data, r.size() * 2);
            for (int32_t k = 0; k < card; ++k) {
                const uint32_t s = r[2 * k], e = std::min<uint32_t>(0xFFFFu, s + r[2 * k + 1]);
                for (uint32_t v = s; v <= e; ++v) g_ids.push_back(base + v);
            }
        } else {
            return CR_ERR_INVALID;
        }
    }
    std::memset(out, 0, sizeof(*out));
    return CR_OK;
}

// Entry points host/api.cpp links against but this program never reaches.
#define STUB(name, ...) \
    int name(__VA_ARGS__) { return CR_ERR_UNSUPPORTED; }
STUB(cr_upload_from_ids, const uint32_t*, uint32_t, uint32_t, cr_stream_t, uint32_t, cr_gpu_roaring*)
STUB(cr_upload_from_device_ids, const uint32_t*, uint32_t, uint32_t, cr_stream_t, uint32_t, cr_gpu_roaring*)
STUB(cr_upload_from_bitset, const uint32_t*, uint32_t, uint32_t, cr_stream_t, cr_gpu_roaring*)
STUB(cr_upload_from_device_bitset, const uint32_t*, uint32_t, uint32_t, cr_stream_t, cr_gpu_roaring*)
STUB(cr_get_meta, const cr_host_container*, uint32_t, cr_meta*)
STUB(cr_set_operation, const cr_gpu_roaring*, const cr_gpu_roaring*, uint32_t, cr_stream_t, cr_gpu_roaring*)
STUB(cr_multi_and, const cr_gpu_roaring*, uint32_t, cr_stream_t, cr_gpu_roaring*)
STUB(cr_free, cr_gpu_roaring*)
STUB(cr_free_async, cr_gpu_roaring*, cr_stream_t)
STUB(cr_resolve_auto_threshold, uint32_t, int, uint32_t*)
STUB(cr_topk_filtered, const float*, uint64_t, const float*, uint32_t, uint32_t, const cr_gpu_roaring*, uint32_t,
     float*, int64_t*, cr_stream_t)
STUB(cr_decompress_to_bitset, const cr_gpu_roaring*, uint32_t*, uint32_t, cr_stream_t)
STUB(cr_decompress_to_bitset_alloc, const cr_gpu_roaring*, cr_stream_t, uint32_t**, uint32_t*)
STUB(cr_enumerate_ids, const cr_gpu_roaring*, int64_t*, uint64_t, cr_stream_t)
STUB(cr_enumerate_ids_alloc, const cr_gpu_roaring*, cr_stream_t, int64_t**, uint64_t*)
STUB(cr_cardinality, const cr_gpu_roaring*, cr_stream_t, uint64_t*)
STUB(cr_promote_to_bitmap, const cr_gpu_roaring*, cr_stream_t, cr_gpu_roaring*)
STUB(cr_promote_auto, const cr_gpu_roaring*, cr_stream_t, int, cr_gpu_roaring*)
STUB(cr_deep_copy, const cr_gpu_roaring*, cr_stream_t, cr_gpu_roaring*)
STUB(cr_portable_size_in_bytes, const cr_gpu_roaring*, cr_stream_t, size_t*)
STUB(cr_portable_serialize, const cr_gpu_roaring*, cr_stream_t, void*, size_t, size_t*)
}  // extern "C"

static std::vector<uint8_t> read_file(const std::string& p)
{
    std::ifstream f(p, std::ios::binary);
    return std::vector<uint8_t>((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
}

// Parses `data` (copied into an allocation of exactly its size, so ASan sees
// any read past it); returns the status.
static int parse(const std::vector<uint8_t>& data, uint32_t universe)
{
    std::vector<uint8_t> exact(data);
    cr_gpu_roaring out;
    return cr_portable_deserialize(exact.empty() ? nullptr : exact.data(), exact.size(), universe, nullptr,
                                   CR_PROMOTE_KEEP_DEFAULT, &out);
}

int main(int argc, char** argv)
{
    if (argc != 2) {
        std::printf("usage: host_sanitize DIR\n");
        return 2;
    }
    std::mt19937 gen(12345);
    int cases = 0;
    for (int i = 0;; ++i) {
        const std::string base = std::string(argv[1]) + "/case_" + std::to_string(i);
        const std::vector<uint8_t> bin = read_file(base + ".bin"), raw = read_file(base + ".ids");
        if (raw.size() < 4) break;
        ++cases;
        uint32_t universe;
        std::memcpy(&universe, raw.data(), 4);
        std::vector<uint32_t> ids((raw.size() - 4) / 4);
        if (!ids.empty()) std::memcpy(ids.data(), raw.data() + 4, ids.size() * 4);
        // the parse hands over exactly the set
        CHECK(parse(bin, 0) == CR_OK && !g_complemented && g_ids == ids);
        // upload(bm, U): more than U/2 ids -> the complement within [0, U)
        if (universe) {
            CHECK(parse(bin, universe) == CR_OK && g_universe == universe);
            const bool over = ids.size() > universe / 2u;
            CHECK(g_complemented == over);
            if (over) {
                std::vector<uint32_t> all(g_ids);
                all.insert(all.end(), ids.begin(), ids.end());
                std::sort(all.begin(), all.end());
                bool ok = all.size() == universe;
                for (uint32_t v = 0; ok && v < universe; ++v) ok = all[v] == v;
                CHECK(ok);
            } else {
                CHECK(g_ids == ids);
            }
        }
        // mutations: rejected, or parsed into well-formed containers
        for (int m = 0; m < 3000; ++m) {
            std::vector<uint8_t> d(bin);
            const int kind = static_cast<int>(gen() % 4);
            if (kind == 0 && !d.empty()) {
                for (int f = 0, nf = 1 + static_cast<int>(gen() % 4); f < nf; ++f)
                    d[gen() % d.size()] ^= static_cast<uint8_t>(1u << (gen() % 8));
            } else if (kind == 1 && !d.empty()) {
                d.resize(gen() % d.size());
            } else if (kind == 2) {
                const size_t hdr = std::min<size_t>(d.size(), 64);
                if (hdr) d[gen() % hdr] = static_cast<uint8_t>(gen());
            } else {
                for (int e = 0, ne = 1 + static_cast<int>(gen() % 64); e < ne; ++e) d.push_back(static_cast<uint8_t>(gen()));
            }
            // The format leaves payload contents unchecked (an array's values
            // need not be sorted); what the parse must guarantee is that every
            // container it hands over lies inside the input, which the decode
            // of each one, under ASan, checks.
            const int rc = parse(d, (m & 1) ? universe : 0u);
            CHECK(rc == CR_OK || rc == CR_ERR_INVALID);
        }
    }
    CHECK(cases > 0);
    if (g_fail) {
        std::printf("host_sanitize: %d check(s) failed over %d cases\n", g_fail, cases);
        return 1;
    }
    std::printf("host_sanitize: OK (%d cases, %d parses handed over)\n", cases, g_uploads);
    return 0;
}

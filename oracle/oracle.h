/*
 * oracle.h -- CPU restatement of cu-roaring-bitmap's hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
 * calls this code.  It is used by tests/ (as the checker), by
 * __graft_entry__.smoke() (as the checker) and by bench.py's cpu_baseline leg
 * (as the timed CPU port).  Every function cites the reference file:line whose
 * behaviour it restates (paths are relative to the reference checkout).
 *
 * Three parts:
 *   1. ref-semantics  -- the reference's *output layout* rules for the GPU
 *      structs (upload_from_ids, bitset uploads, packed upload(), set_operation,
 *      multi_and, resolve_auto_threshold, contains, decompress, enumerate_ids,
 *      promote_to_bitmap, deep copy).
 *   2. roaring-lite   -- a host Roaring bitmap with array / bitset / run
 *      containers following the public Roaring format rules (array <= 4096,
 *      run chosen iff its serialized size is smaller).  It stands in for
 *      CRoaring, which is absent: inputs for upload(), the logical oracle for
 *      set operations, and the CPU baseline.
 *   3. generators     -- MT19937 and libstdc++'s generate_canonical<double>,
 *      so the reference tests' std::mt19937 inputs can be regenerated, and the
 *      splitmix64 counter hash used for the benchmark inputs.
 *
 * Pinning (which check fixes which function) is listed in the header comment
 * of each .c file and in tests/test_oracle_*.py.
 */
#ifndef CR_ORACLE_H
#define CR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ContainerType (include/cu_roaring/types.cuh:7-11). */
enum { ORC_ARRAY = 0, ORC_BITMAP = 1, ORC_RUN = 2 };
/* SetOp (include/cu_roaring/detail/set_ops.cuh:7-12). */
enum { ORC_AND = 0, ORC_OR = 1, ORC_ANDNOT = 2, ORC_XOR = 3 };
/* PROMOTE_* (include/cu_roaring/detail/promote.cuh:38-40). */
#define ORC_PROMOTE_KEEP_DEFAULT 4096u
#define ORC_PROMOTE_ALL 0u
#define ORC_PROMOTE_AUTO 0xFFFFFFFFu
/* CRoaring type codes used by upload() (src/upload.cpp:21-23). */
enum { ORC_TC_BITSET = 1, ORC_TC_ARRAY = 2, ORC_TC_RUN = 3 };

/*
 * Host mirror of GpuRoaring (include/cu_roaring/types.cuh:15-54).  Pools are
 * host arrays; bitmap_pool_words / key_index_len record the allocated sizes so
 * a "strict layout" comparison can include pool holes.
 */
typedef struct orc_roaring {
    uint16_t* keys;
    uint8_t* types;
    uint32_t* offsets; /* BYTE offsets into the per-type pool */
    uint16_t* cards;
    uint32_t n_containers;
    uint32_t universe_size;
    uint64_t total_cardinality;
    uint64_t* bitmap_data;
    uint32_t n_bitmap_containers;
    uint32_t bitmap_pool_words;
    uint16_t* array_data;
    uint32_t n_array_containers;
    uint32_t array_pool_bytes;
    uint16_t* run_data;
    uint32_t n_run_containers;
    uint32_t run_pool_bytes;
    uint16_t* key_index; /* NULL when absent */
    uint32_t key_index_len;
    uint32_t max_key;
    int32_t negated;
} orc_roaring;

/* One CRoaring-style container handed to the packed upload(). */
typedef struct orc_container {
    uint16_t key;
    uint8_t typecode; /* ORC_TC_* */
    int32_t card;     /* bitset: cardinality 0..65536; array: cardinality; run: n_runs */
    const void* data; /* bitset: 1024 u64; array: card u16; run: n_runs (start,length) u16 pairs */
} orc_container;

void orc_free(orc_roaring* r);

/* ---- ref-semantics ------------------------------------------------------ */
uint32_t orc_resolve_auto_threshold(uint32_t universe_size, uint64_t l2_bytes);
int orc_upload_from_ids(const uint32_t* ids, uint32_t n_ids, uint32_t universe_size,
                        uint32_t bitmap_threshold, uint64_t l2_bytes, orc_roaring* out);
int orc_upload_from_bitset(const uint32_t* words, uint32_t n_words, uint32_t universe_size,
                           orc_roaring* out);
int orc_upload_packed(const orc_container* conts, uint32_t n, uint32_t explicit_universe,
                      int complement_applied, uint64_t logical_card, uint32_t bitmap_threshold,
                      uint64_t l2_bytes, orc_roaring* out);
int orc_set_operation(const orc_roaring* a, const orc_roaring* b, int op, orc_roaring* out);
int orc_multi_and(const orc_roaring* inputs, uint32_t count, orc_roaring* out);
int orc_contains(const orc_roaring* r, uint32_t id);
void orc_contains_many(const orc_roaring* r, const uint32_t* ids, uint64_t n, uint32_t* out);
void orc_decompress(const orc_roaring* r, uint32_t* out_words, uint32_t n_words);
uint64_t orc_true_cardinality(const orc_roaring* r);
uint64_t orc_enumerate_ids(const orc_roaring* r, int64_t* out);
int orc_promote_to_bitmap(const orc_roaring* src, orc_roaring* out);
int orc_deep_copy(const orc_roaring* src, orc_roaring* out);

/* ---- roaring-lite ------------------------------------------------------- */
typedef struct rl_bitmap {
    uint32_t n;
    uint32_t cap;
    uint16_t* keys;
    uint8_t* tc;     /* ORC_TC_* */
    int32_t* card;   /* bitset/array: cardinality; run: n_runs */
    void** data;
} rl_bitmap;

rl_bitmap* rl_create(void);
void rl_destroy(rl_bitmap* b);
rl_bitmap* rl_from_sorted_ids(const uint32_t* ids, uint64_t n); /* sorted, unique */
rl_bitmap* rl_from_ids(const uint32_t* ids, uint64_t n);        /* any order, dups ok */
rl_bitmap* rl_from_words(const uint64_t* words, uint64_t n_words); /* flat bitset, bit i = id i */
rl_bitmap* rl_copy(const rl_bitmap* b);
void rl_run_optimize(rl_bitmap* b);
rl_bitmap* rl_op(const rl_bitmap* a, const rl_bitmap* b, int op);
rl_bitmap* rl_flip(const rl_bitmap* b, uint64_t lo, uint64_t hi);
rl_bitmap* rl_slice(const rl_bitmap* b, uint32_t key_lo, uint32_t key_hi); /* keys in [lo, hi), copied */
int rl_contains(const rl_bitmap* b, uint32_t id);
void rl_contains_many(const rl_bitmap* b, const uint32_t* ids, uint64_t n, uint32_t* out);
uint64_t rl_cardinality(const rl_bitmap* b);
uint64_t rl_to_ids(const rl_bitmap* b, uint32_t* out); /* out may be NULL: count only */
uint32_t rl_n_containers(const rl_bitmap* b);
void rl_container_info(const rl_bitmap* b, uint32_t i, uint16_t* key, uint8_t* tc, int32_t* card,
                       const void** data);
void rl_to_containers(const rl_bitmap* b, orc_container* out);
void rl_count_types(const rl_bitmap* b, uint32_t* n_bitset, uint32_t* n_array, uint32_t* n_run);
/* Roaring portable format (roaring_lite.c documents the layout). */
uint64_t rl_portable_size(const rl_bitmap* b);
uint64_t rl_portable_serialize(const rl_bitmap* b, uint8_t* out);
rl_bitmap* rl_portable_deserialize(const uint8_t* buf, uint64_t len, uint64_t* consumed);

/* ---- generators --------------------------------------------------------- */
typedef struct orc_mt19937 {
    uint32_t mt[624];
    uint32_t idx;
} orc_mt19937;
void orc_mt_seed(orc_mt19937* g, uint32_t seed);
uint32_t orc_mt_next(orc_mt19937* g);
double orc_mt_canonical(orc_mt19937* g);
/* Fill out[i] = 1 when std::uniform_real_distribution<double>(0,1)(gen) < density, i in [0,n). */
void orc_mt_bernoulli_ids(uint32_t seed, double density, uint32_t universe, uint32_t* out_ids,
                          uint64_t* out_n);
void orc_mt_raw(uint32_t seed, uint32_t* out, uint64_t n);
uint64_t orc_splitmix64(uint64_t x);

/* ---- CPU brute force top-k (fp64 distances) ------------------------------ */
void orc_topk_bruteforce(const float* base, uint64_t n_base, const float* queries, uint32_t n_q,
                         uint32_t dim, const uint8_t* pass, uint32_t k, double* out_dist,
                         int64_t* out_ids, int n_threads);

/* ---- CPU baselines timed by bench.py (cpu_baseline.c) --------------------
 * Each returns the seconds of its timed work; threads >= 1. */
double orc_cpu_upload_ids(const uint32_t* ids, uint64_t n, uint32_t universe, int threads, orc_roaring* out);
double orc_cpu_setop(const rl_bitmap* const* a_shards, const rl_bitmap* const* b_shards, uint32_t n_shards, int op,
                     int threads, uint64_t* out_card, uint64_t* out_containers);
double orc_cpu_multi_and(const rl_bitmap* const* inputs, uint32_t k, uint32_t n_shards, int threads,
                         uint64_t* out_card, uint64_t* out_containers);
double orc_cpu_contains(const rl_bitmap* b, const uint32_t* q, uint64_t n, uint32_t* out, int threads);
double orc_cpu_config0(const uint32_t* a_ids, uint64_t na, const uint32_t* b_ids, uint64_t nb, const uint32_t* q,
                       uint64_t nq, double* t_parts, uint64_t* cards, uint64_t* hits);
double orc_cpu_topk_fp32(const float* base, uint64_t n_base, const float* queries, uint32_t n_q, uint32_t dim,
                         const uint8_t* pass, uint32_t k, float* out_dist, int64_t* out_ids, int threads);

#ifdef __cplusplus
}
#endif
#endif /* CR_ORACLE_H */

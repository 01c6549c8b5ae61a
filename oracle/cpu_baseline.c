/*
 * cpu_baseline.c -- the CPU side that bench.py times beside the GPU (its
 * cpu_baseline leg).  BENCH/TEST INFRASTRUCTURE ONLY: the product library
 * never links, loads or calls it.
 *
 * The reference's CPU path is CRoaring (third_party/CRoaring, absent from the
 * checkout) plus std::sort + unique for the id upload
 * (bench/bench_upload_scale.cu:102-125, bench/bench_multi_and.cu:144-156,
 * bench/bench_set_ops.cu:43-60).  These functions time the same work with
 * roaring-lite's CRoaring-equivalent algorithms (merge / galloping array
 * intersection, word-wise bitset ops with popcount), at 1 thread -- CRoaring is
 * single-threaded -- and at T threads, sharded by container key range or by
 * query.  Each returns the seconds of its own timed work (CLOCK_MONOTONIC),
 * which excludes input preparation and the freeing of results.
 *
 * Pinning (tests/test_oracle_cpu_baseline.py): every function's output is
 * compared with the single-threaded oracle on the same input --
 * orc_cpu_upload_ids with orc_upload_from_ids (all fields, strict);
 * orc_cpu_setop / orc_cpu_multi_and with rl_op over the whole bitmaps
 * (cardinalities and decoded ids); orc_cpu_contains with rl_contains_many;
 * orc_cpu_topk_fp32 with the fp64 brute force orc_topk_bruteforce (1e-4
 * relative, id sets equal except at ties); orc_cpu_config0 with numpy sets.
 */
#define _POSIX_C_SOURCE 200809L
#include "oracle.h"

#include <immintrin.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static double now_s(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

typedef void* (*worker_fn)(void*);

/* Run fn(arg_i) on `threads` threads; arg_i = base + i * stride bytes. */
static void run_threads(int threads, worker_fn fn, void* base, size_t stride)
{
    if (threads <= 1) {
        fn(base);
        return;
    }
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    for (int t = 0; t < threads; ++t) pthread_create(&th[t], NULL, fn, (char*)base + (size_t)t * stride);
    for (int t = 0; t < threads; ++t) pthread_join(th[t], NULL);
    free(th);
}

/* ==========================================================================
 * upload from ids, threaded: the all-bitmap layout of the reference's GPU
 * path (src/upload_ids.cu:171-416, as orc_upload_from_ids restates it) built
 * by a bucket partition instead of a sort: ids are split into R key ranges
 * (count, scatter), then each range's containers are filled by setting bits,
 * popcounted, and ranked.  Inputs that would be stored as a complement
 * (distinct ids > U/2) are rejected: the bench's inputs are not.
 * ========================================================================== */
typedef struct {
    const uint32_t* ids;
    uint64_t n;
    uint32_t K, R, kpr, T;
    uint64_t* cnt; /* [T][R] */
    uint64_t* off; /* [T][R] */
    uint32_t* part;
    uint64_t* pool; /* K x 1024, key-addressed */
    uint32_t* key_cnt;
    volatile int next_range;
    int phase;
    int bad;
} up_ctx;

typedef struct {
    up_ctx* c;
    uint32_t t;
} up_arg;

static void* up_worker(void* p)
{
    up_arg* a = (up_arg*)p;
    up_ctx* c = a->c;
    const uint64_t lo = c->n * a->t / c->T, hi = c->n * (a->t + 1) / c->T;
    if (c->phase == 0) {
        uint64_t* cnt = c->cnt + (size_t)a->t * c->R;
        for (uint64_t i = lo; i < hi; ++i) {
            const uint32_t key = c->ids[i] >> 16;
            if (key >= c->K) {
                c->bad = 1;
                continue;
            }
            ++cnt[key / c->kpr];
        }
    } else if (c->phase == 1) {
        uint64_t* off = c->off + (size_t)a->t * c->R;
        for (uint64_t i = lo; i < hi; ++i) {
            const uint32_t key = c->ids[i] >> 16;
            if (key < c->K) c->part[off[key / c->kpr]++] = c->ids[i];
        }
    } else {
        for (;;) {
            const uint32_t r = (uint32_t)__atomic_fetch_add(&c->next_range, 1, __ATOMIC_RELAXED);
            if (r >= c->R) break;
            const uint32_t k0 = r * c->kpr, k1 = k0 + c->kpr < c->K ? k0 + c->kpr : c->K;
            uint64_t* base = c->pool + (size_t)k0 * 1024u;
            memset(base, 0, (size_t)(k1 - k0) * 8192u);
            /* the range's ids: from its start in thread 0's slice to its end in the last thread's */
            const uint64_t s = c->off[r] - c->cnt[r];
            const uint64_t e = c->off[(size_t)(c->T - 1) * c->R + r];
            for (uint64_t i = s; i < e; ++i) {
                const uint32_t id = c->part[i];
                const uint32_t w = ((id >> 16) - k0) * 1024u + ((id & 0xFFFFu) >> 6);
                base[w] |= 1ull << (id & 63u);
            }
            for (uint32_t k = k0; k < k1; ++k) {
                const uint64_t* b = c->pool + (size_t)k * 1024u;
                uint32_t pc = 0;
                for (uint32_t w = 0; w < 1024u; ++w) pc += (uint32_t)__builtin_popcountll(b[w]);
                c->key_cnt[k] = pc;
            }
        }
    }
    return NULL;
}

double orc_cpu_upload_ids(const uint32_t* ids, uint64_t n, uint32_t universe, int threads, orc_roaring* out)
{
    memset(out, 0, sizeof(*out));
    if (threads < 1) threads = 1;
    uint32_t max_key = universe ? (universe - 1u) >> 16 : 0u;
    if (max_key > 0xFFFFu) max_key = 0xFFFFu;
    const uint32_t K = max_key + 1u;
    const double t0 = now_s();
    up_ctx c;
    memset(&c, 0, sizeof(c));
    c.ids = ids;
    c.n = n;
    c.K = K;
    c.T = (uint32_t)threads;
    c.R = K < 4096u ? K : 4096u;
    c.kpr = (K + c.R - 1) / c.R;
    c.R = (K + c.kpr - 1) / c.kpr;
    c.cnt = (uint64_t*)calloc((size_t)c.T * c.R, 8);
    c.off = (uint64_t*)malloc((size_t)c.T * c.R * 8);
    c.part = (uint32_t*)malloc((size_t)(n ? n : 1) * 4u);
    c.pool = (uint64_t*)malloc((size_t)K * 8192u);
    c.key_cnt = (uint32_t*)malloc((size_t)K * 4u);
    up_arg* args = (up_arg*)malloc(sizeof(up_arg) * c.T);
    for (uint32_t t = 0; t < c.T; ++t) args[t] = (up_arg){&c, t};
    c.phase = 0;
    run_threads(threads, up_worker, args, sizeof(up_arg));
    uint64_t acc = 0; /* range-major, thread-minor starts */
    for (uint32_t r = 0; r < c.R; ++r)
        for (uint32_t t = 0; t < c.T; ++t) {
            c.off[(size_t)t * c.R + r] = acc;
            acc += c.cnt[(size_t)t * c.R + r];
        }
    c.phase = 1;
    run_threads(threads, up_worker, args, sizeof(up_arg));
    /* after the scatter off[t][r] is the end of slice (t, r): off[0][r] - cnt[0][r] is the range's start */
    c.phase = 2;
    c.next_range = 0;
    run_threads(threads, up_worker, args, sizeof(up_arg));
    /* ranks of the present keys, then the metadata (src/upload_ids.cu:26-106,255-295) */
    uint32_t n_c = 0;
    uint64_t total = 0;
    for (uint32_t k = 0; k < K; ++k) {
        n_c += c.key_cnt[k] != 0;
        total += c.key_cnt[k];
    }
    /* a key past max_key, or a set that would be stored as its complement */
    const int ok = !c.bad && total <= (uint64_t)universe / 2u;
    if (ok) {
        out->universe_size = universe;
        out->total_cardinality = total;
        out->n_containers = out->n_bitmap_containers = n_c;
        out->max_key = max_key;
        out->key_index_len = K;
        out->bitmap_pool_words = n_c * 1024u;
        out->keys = (uint16_t*)malloc((size_t)(n_c ? n_c : 1) * 2u);
        out->types = (uint8_t*)malloc(n_c ? n_c : 1);
        out->offsets = (uint32_t*)malloc((size_t)(n_c ? n_c : 1) * 4u);
        out->cards = (uint16_t*)malloc((size_t)(n_c ? n_c : 1) * 2u);
        out->key_index = (uint16_t*)malloc((size_t)K * 2u);
        uint32_t i = 0;
        for (uint32_t k = 0; k < K; ++k) {
            if (!c.key_cnt[k]) {
                out->key_index[k] = 0xFFFFu;
                continue;
            }
            out->keys[i] = (uint16_t)k;
            out->types[i] = ORC_BITMAP;
            out->offsets[i] = i * 8192u;
            out->cards[i] = (uint16_t)(c.key_cnt[k] > 65535u ? 0u : c.key_cnt[k]);
            out->key_index[k] = (uint16_t)i;
            if (i != k) memmove(c.pool + (size_t)i * 1024u, c.pool + (size_t)k * 1024u, 8192u); /* i < k */
            ++i;
        }
        out->bitmap_data = c.pool;
        c.pool = NULL;
    }
    const double dt = now_s() - t0;
    free(args);
    free(c.cnt);
    free(c.off);
    free(c.part);
    free(c.pool);
    free(c.key_cnt);
    return ok ? dt : -1.0;
}

/* ==========================================================================
 * set operations and multi_and, sharded by key range.  shards[i] are the
 * containers of one key range of an operand (rl_slice); a worker takes shards
 * in turn and computes rl_op (and its cardinality) on them.  The CPU
 * multi_and is the reference's: a copy of the first input ANDed in place with
 * each other one (bench/bench_multi_and.cu:144-156).
 * ========================================================================== */
typedef struct {
    const rl_bitmap* const* a;
    const rl_bitmap* const* b;
    uint32_t k; /* multi_and inputs (0: a set operation on a, b) */
    uint32_t n_shards;
    int op;
    rl_bitmap** res;
    uint64_t* card;
    volatile int next;
} so_ctx;

static void* so_worker(void* p)
{
    so_ctx* c = *(so_ctx**)p;
    for (;;) {
        const uint32_t s = (uint32_t)__atomic_fetch_add(&c->next, 1, __ATOMIC_RELAXED);
        if (s >= c->n_shards) break;
        rl_bitmap* r;
        if (c->k == 0) {
            r = rl_op(c->a[s], c->b[s], c->op);
        } else {
            r = rl_op(c->a[s], c->a[(size_t)c->n_shards + s], ORC_AND);
            for (uint32_t j = 2; j < c->k; ++j) {
                rl_bitmap* x = rl_op(r, c->a[(size_t)j * c->n_shards + s], ORC_AND);
                rl_destroy(r);
                r = x;
            }
        }
        c->card[s] = rl_cardinality(r);
        c->res[s] = r;
    }
    return NULL;
}

static double so_run(so_ctx* c, int threads, uint64_t* out_card, uint64_t* out_containers)
{
    c->res = (rl_bitmap**)calloc(c->n_shards, sizeof(rl_bitmap*));
    c->card = (uint64_t*)calloc(c->n_shards, 8);
    c->next = 0;
    if (threads < 1) threads = 1;
    so_ctx** args = (so_ctx**)malloc(sizeof(so_ctx*) * (size_t)threads);
    for (int t = 0; t < threads; ++t) args[t] = c;
    const double t0 = now_s();
    run_threads(threads, so_worker, args, sizeof(so_ctx*));
    const double dt = now_s() - t0;
    uint64_t card = 0, nc = 0;
    for (uint32_t s = 0; s < c->n_shards; ++s) {
        card += c->card[s];
        nc += c->res[s]->n;
        rl_destroy(c->res[s]);
    }
    if (out_card) *out_card = card;
    if (out_containers) *out_containers = nc;
    free(args);
    free(c->res);
    free(c->card);
    return dt;
}

double orc_cpu_setop(const rl_bitmap* const* a_shards, const rl_bitmap* const* b_shards, uint32_t n_shards, int op,
                     int threads, uint64_t* out_card, uint64_t* out_containers)
{
    so_ctx c;
    memset(&c, 0, sizeof(c));
    c.a = a_shards;
    c.b = b_shards;
    c.n_shards = n_shards;
    c.op = op;
    return so_run(&c, threads, out_card, out_containers);
}

/* inputs[j * n_shards + s] is shard s of input j, for k >= 2 inputs. */
double orc_cpu_multi_and(const rl_bitmap* const* inputs, uint32_t k, uint32_t n_shards, int threads,
                         uint64_t* out_card, uint64_t* out_containers)
{
    so_ctx c;
    memset(&c, 0, sizeof(c));
    c.a = inputs;
    c.k = k < 2 ? 2 : k;
    c.n_shards = n_shards;
    return so_run(&c, threads, out_card, out_containers);
}

/* ==========================================================================
 * contains, sharded by query: rl_contains (a binary search over the keys,
 * then the container's own search) per query.
 * ========================================================================== */
typedef struct {
    const rl_bitmap* b;
    const uint32_t* q;
    uint32_t* out;
    uint64_t lo, hi;
} ct_arg;

static void* ct_worker(void* p)
{
    ct_arg* a = (ct_arg*)p;
    rl_contains_many(a->b, a->q + a->lo, a->hi - a->lo, a->out + a->lo);
    return NULL;
}

double orc_cpu_contains(const rl_bitmap* b, const uint32_t* q, uint64_t n, uint32_t* out, int threads)
{
    if (threads < 1) threads = 1;
    ct_arg* args = (ct_arg*)malloc(sizeof(ct_arg) * (size_t)threads);
    for (int t = 0; t < threads; ++t)
        args[t] = (ct_arg){b, q, out, n * (uint64_t)t / (uint64_t)threads, n * (uint64_t)(t + 1) / (uint64_t)threads};
    const double t0 = now_s();
    run_threads(threads, ct_worker, args, sizeof(ct_arg));
    const double dt = now_s() - t0;
    free(args);
    return dt;
}

/* ==========================================================================
 * two bitmaps over 2^24 built from ids, AND/OR/ANDNOT/XOR with
 * their cardinalities, then point queries -- one thread, as CRoaring runs it.
 * t_parts: build, the four operations, the queries.
 * ========================================================================== */
double orc_cpu_config0(const uint32_t* a_ids, uint64_t na, const uint32_t* b_ids, uint64_t nb, const uint32_t* q,
                       uint64_t nq, double* t_parts, uint64_t* cards, uint64_t* hits)
{
    const double t0 = now_s();
    rl_bitmap* a = rl_from_ids(a_ids, na);
    rl_bitmap* b = rl_from_ids(b_ids, nb);
    const double t1 = now_s();
    rl_bitmap* r[4];
    for (int op = 0; op < 4; ++op) {
        r[op] = rl_op(a, b, op);
        cards[op] = rl_cardinality(r[op]);
    }
    const double t2 = now_s();
    uint64_t h = 0;
    for (uint64_t i = 0; i < nq; ++i) h += (uint64_t)rl_contains(a, q[i]);
    const double t3 = now_s();
    *hits = h;
    t_parts[0] = t1 - t0;
    t_parts[1] = t2 - t1;
    t_parts[2] = t3 - t2;
    for (int op = 0; op < 4; ++op) rl_destroy(r[op]);
    rl_destroy(a);
    rl_destroy(b);
    return t3 - t0;
}

/* ==========================================================================
 * filtered brute-force top-k in fp32: each worker takes blocks of TQ queries
 * and scans the passing base rows in blocks of TR, computing the direct
 * squared L2 distance sum((q - x)^2) in eight AVX2 partial sums per pair
 * (x86-64-v3, the oracle's build target), and keeps each query's
 * k best by (distance, id) in a max-heap.  Rows are visited in id order and a
 * row enters only if strictly better than the heap's worst, so on equal
 * distances the smaller id stays, as in the GPU kernel and the fp64 oracle.
 * ========================================================================== */
#define TK_TQ 8
#define TK_TR 64

typedef struct {
    const float* base;
    uint64_t n_base;
    const float* q;
    uint32_t n_q, dim, k;
    const uint8_t* pass;
    float* out_d;
    int64_t* out_i;
    volatile int next;
} tk_ctx;

static int tk_worse(float da, int64_t ia, float db, int64_t ib) { return da > db || (da == db && ia > ib); }

static void heap_sift_down(float* d, int64_t* id, uint32_t n, uint32_t i)
{
    for (;;) {
        uint32_t l = 2 * i + 1, m = i;
        if (l < n && tk_worse(d[l], id[l], d[m], id[m])) m = l;
        if (l + 1 < n && tk_worse(d[l + 1], id[l + 1], d[m], id[m])) m = l + 1;
        if (m == i) return;
        float td = d[i];
        d[i] = d[m];
        d[m] = td;
        int64_t ti = id[i];
        id[i] = id[m];
        id[m] = ti;
        i = m;
    }
}

/* Squared L2 distances of one row x to the TK_TQ queries q[0..nq): eight fp32
 * lanes of AVX2 per query, one FMA chain per query (independent chains, so
 * they overlap), the lanes summed pairwise at the end. */
static void dist_block(const float* const* q, uint32_t nq, const float* x, uint32_t dim, float* out)
{
    __m256 acc[TK_TQ];
    for (uint32_t j = 0; j < TK_TQ; ++j) acc[j] = _mm256_setzero_ps();
    uint32_t d = 0;
    for (; d + 8 <= dim; d += 8) {
        const __m256 xv = _mm256_loadu_ps(x + d);
        for (uint32_t j = 0; j < nq; ++j) {
            const __m256 t = _mm256_sub_ps(_mm256_loadu_ps(q[j] + d), xv);
            acc[j] = _mm256_fmadd_ps(t, t, acc[j]);
        }
    }
    for (uint32_t j = 0; j < nq; ++j) {
        float a[8];
        _mm256_storeu_ps(a, acc[j]);
        for (uint32_t e = d; e < dim; ++e) {
            const float t = q[j][e] - x[e];
            a[e & 7] += t * t;
        }
        out[j] = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
    }
}

static void* tk_worker(void* p)
{
    tk_ctx* c = *(tk_ctx**)p;
    const uint32_t k = c->k;
    float* hd = (float*)malloc(sizeof(float) * TK_TQ * k);
    int64_t* hi = (int64_t*)malloc(sizeof(int64_t) * TK_TQ * k);
    uint32_t fill[TK_TQ];
    for (;;) {
        const uint32_t q0 = (uint32_t)__atomic_fetch_add(&c->next, TK_TQ, __ATOMIC_RELAXED);
        if (q0 >= c->n_q) break;
        const uint32_t nq = c->n_q - q0 < TK_TQ ? c->n_q - q0 : TK_TQ;
        const float* qp[TK_TQ];
        for (uint32_t j = 0; j < nq; ++j) {
            fill[j] = 0;
            qp[j] = c->q + (size_t)(q0 + j) * c->dim;
        }
        for (uint64_t r0 = 0; r0 < c->n_base; r0 += TK_TR) {
            const uint64_t r1 = r0 + TK_TR < c->n_base ? r0 + TK_TR : c->n_base;
            for (uint64_t r = r0; r < r1; ++r) {
                if (c->pass && !c->pass[r]) continue;
                const float* x = c->base + r * c->dim;
                float dv[TK_TQ];
                dist_block(qp, nq, x, c->dim, dv);
                for (uint32_t j = 0; j < nq; ++j) {
                    const float dd = dv[j];
                    float* d = hd + (size_t)j * k;
                    int64_t* id = hi + (size_t)j * k;
                    if (fill[j] < k) { /* sift up */
                        uint32_t i = fill[j]++;
                        d[i] = dd;
                        id[i] = (int64_t)r;
                        while (i > 0 && tk_worse(d[i], id[i], d[(i - 1) / 2], id[(i - 1) / 2])) {
                            const uint32_t pnt = (i - 1) / 2;
                            float td = d[i];
                            d[i] = d[pnt];
                            d[pnt] = td;
                            int64_t ti = id[i];
                            id[i] = id[pnt];
                            id[pnt] = ti;
                            i = pnt;
                        }
                    } else if (dd < d[0]) {
                        d[0] = dd;
                        id[0] = (int64_t)r;
                        heap_sift_down(d, id, k, 0);
                    }
                }
            }
        }
        for (uint32_t j = 0; j < nq; ++j) { /* heap -> ascending (distance, id); unfilled slots (+inf, -1) */
            float* d = hd + (size_t)j * k;
            int64_t* id = hi + (size_t)j * k;
            float* od = c->out_d + (size_t)(q0 + j) * k;
            int64_t* oi = c->out_i + (size_t)(q0 + j) * k;
            for (uint32_t s = fill[j]; s < k; ++s) {
                od[s] = __builtin_inff();
                oi[s] = -1;
            }
            for (uint32_t n = fill[j]; n > 0; --n) {
                od[n - 1] = d[0];
                oi[n - 1] = id[0];
                d[0] = d[n - 1];
                id[0] = id[n - 1];
                heap_sift_down(d, id, n - 1, 0);
            }
        }
    }
    free(hd);
    free(hi);
    return NULL;
}

double orc_cpu_topk_fp32(const float* base, uint64_t n_base, const float* queries, uint32_t n_q, uint32_t dim,
                         const uint8_t* pass, uint32_t k, float* out_dist, int64_t* out_ids, int threads)
{
    if (threads < 1) threads = 1;
    tk_ctx c = {base, n_base, queries, n_q, dim, k, pass, out_dist, out_ids, 0};
    tk_ctx** args = (tk_ctx**)malloc(sizeof(tk_ctx*) * (size_t)threads);
    for (int t = 0; t < threads; ++t) args[t] = &c;
    const double t0 = now_s();
    run_threads(threads, tk_worker, args, sizeof(tk_ctx*));
    const double dt = now_s() - t0;
    free(args);
    return dt;
}

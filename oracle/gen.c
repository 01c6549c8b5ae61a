/*
 * gen.c -- input generators and the brute-force top-k (TEST INFRASTRUCTURE ONLY).
 *
 * MT19937 follows the published algorithm (Matsumoto & Nishimura 1998) with the
 * init_genrand seeding that std::mt19937(seed) uses; orc_mt_canonical restates
 * libstdc++'s generate_canonical<double, 53> for a 32-bit engine (two draws,
 * (d0 + d1 * 2^32) / 2^64).  Together they regenerate the inputs of the
 * reference tests that draw with std::mt19937 + uniform_real_distribution
 * (e.g. test/test_set_ops.cu:15-25, test/test_complement.cu:372-380).
 * Pinned by tests/test_oracle_gen.py: the 10000th output of mt19937(5489) is
 * 4123659995 (C++11 [rand.predef]), plus first outputs for seed 5489.
 *
 * orc_topk_bruteforce is the closed-form oracle of the filtered top-k: exact
 * fp64 squared-L2 distances over the passing set, partial selection of the k
 * smallest with ties broken by the smaller id.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

void orc_mt_seed(orc_mt19937* g, uint32_t seed)
{
    g->mt[0] = seed;
    for (uint32_t i = 1; i < 624; ++i)
        g->mt[i] = 1812433253u * (g->mt[i - 1] ^ (g->mt[i - 1] >> 30)) + i;
    g->idx = 624;
}

uint32_t orc_mt_next(orc_mt19937* g)
{
    if (g->idx >= 624) {
        for (uint32_t i = 0; i < 624; ++i) {
            uint32_t y = (g->mt[i] & 0x80000000u) | (g->mt[(i + 1) % 624] & 0x7fffffffu);
            uint32_t v = g->mt[(i + 397) % 624] ^ (y >> 1);
            if (y & 1u) v ^= 0x9908b0dfu;
            g->mt[i] = v;
        }
        g->idx = 0;
    }
    uint32_t y = g->mt[g->idx++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}

double orc_mt_canonical(orc_mt19937* g)
{
    double d0 = (double)orc_mt_next(g);
    double d1 = (double)orc_mt_next(g);
    double r = (d0 + d1 * 4294967296.0) / 18446744073709551616.0;
    if (r >= 1.0) r = nextafter(1.0, 0.0);
    return r;
}

void orc_mt_bernoulli_ids(uint32_t seed, double density, uint32_t universe, uint32_t* out_ids,
                          uint64_t* out_n)
{
    orc_mt19937 g;
    orc_mt_seed(&g, seed);
    uint64_t k = 0;
    for (uint32_t i = 0; i < universe; ++i)
        if (orc_mt_canonical(&g) < density) out_ids[k++] = i;
    *out_n = k;
}

void orc_mt_raw(uint32_t seed, uint32_t* out, uint64_t n)
{
    orc_mt19937 g;
    orc_mt_seed(&g, seed);
    for (uint64_t i = 0; i < n; ++i) out[i] = orc_mt_next(&g);
}

uint64_t orc_splitmix64(uint64_t x)
{
    uint64_t z = x + 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

/* ---- brute-force filtered top-k ---------------------------------------- */
typedef struct {
    const float* base;
    uint64_t n_base;
    const float* queries;
    uint32_t q0, q1, dim, k;
    const uint8_t* pass;
    double* out_dist;
    int64_t* out_ids;
} topk_job;

static int better(double d, int64_t id, double d2, int64_t id2)
{
    return d < d2 || (d == d2 && id < id2);
}

static void* topk_worker(void* arg)
{
    topk_job* j = (topk_job*)arg;
    double* hd = (double*)malloc(sizeof(double) * j->k);
    int64_t* hi = (int64_t*)malloc(sizeof(int64_t) * j->k);
    for (uint32_t q = j->q0; q < j->q1; ++q) {
        const float* qv = j->queries + (size_t)q * j->dim;
        uint32_t cnt = 0; /* sorted insertion list, ascending */
        for (uint64_t i = 0; i < j->n_base; ++i) {
            if (j->pass && !j->pass[i]) continue;
            const float* x = j->base + i * j->dim;
            double d = 0.0;
            for (uint32_t t = 0; t < j->dim; ++t) {
                double df = (double)qv[t] - (double)x[t];
                d += df * df;
            }
            if (cnt == j->k && !better(d, (int64_t)i, hd[cnt - 1], hi[cnt - 1])) continue;
            uint32_t p = cnt < j->k ? cnt++ : cnt - 1;
            while (p > 0 && better(d, (int64_t)i, hd[p - 1], hi[p - 1])) {
                hd[p] = hd[p - 1];
                hi[p] = hi[p - 1];
                --p;
            }
            hd[p] = d;
            hi[p] = (int64_t)i;
        }
        for (uint32_t t = 0; t < j->k; ++t) {
            j->out_dist[(size_t)q * j->k + t] = t < cnt ? hd[t] : INFINITY;
            j->out_ids[(size_t)q * j->k + t] = t < cnt ? hi[t] : -1;
        }
    }
    free(hd);
    free(hi);
    return NULL;
}

void orc_topk_bruteforce(const float* base, uint64_t n_base, const float* queries, uint32_t n_q,
                         uint32_t dim, const uint8_t* pass, uint32_t k, double* out_dist,
                         int64_t* out_ids, int n_threads)
{
    if (n_threads < 1) n_threads = 1;
    if ((uint32_t)n_threads > n_q) n_threads = (int)(n_q ? n_q : 1);
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)n_threads);
    topk_job* jobs = (topk_job*)malloc(sizeof(topk_job) * (size_t)n_threads);
    for (int t = 0; t < n_threads; ++t) {
        jobs[t] = (topk_job){base, n_base, queries, (uint32_t)((uint64_t)n_q * t / n_threads),
                             (uint32_t)((uint64_t)n_q * (t + 1) / n_threads), dim, k, pass, out_dist, out_ids};
        pthread_create(&th[t], NULL, topk_worker, &jobs[t]);
    }
    for (int t = 0; t < n_threads; ++t) pthread_join(th[t], NULL);
    free(th);
    free(jobs);
}

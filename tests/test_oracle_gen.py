"""Pins the oracle's generators (CPU only)."""
import numpy as np

import orc


def test_mt19937_known_answers():
    # C++11 [rand.predef]: the 10000th consecutive invocation of a default-
    # constructed std::mt19937 (seed 5489) produces 4123659995.
    v = orc.mt_raw(5489, 10000)
    assert int(v[-1]) == 4123659995
    # First outputs of mt19937(5489) (published reference output of mt19937ar).
    assert [int(x) for x in v[:5]] == [3499211612, 581869302, 3890346734, 3586334585, 545404204]


def test_canonical_double_matches_two_draw_formula():
    # generate_canonical<double,53> on a 32-bit engine uses two draws:
    # (d0 + d1 * 2^32) / 2^64; density thresholds are applied to that value.
    raw = orc.mt_raw(42, 2 * 1000).astype(np.float64)
    canon = (raw[0::2] + raw[1::2] * 4294967296.0) / 18446744073709551616.0
    ids = orc.mt_bernoulli_ids(42, 0.3, 1000)
    want = np.nonzero(canon < 0.3)[0]
    assert np.array_equal(ids, want)


def test_splitmix64_known_answer():
    # splitmix64 with state 0: first output 0xE220A8397B1DCDAF (Vigna's reference).
    assert orc.splitmix64(0) == 0xE220A8397B1DCDAF


def _topk_numpy(base, queries, k, passing):
    """Independent closed form: full fp64 distance matrix, lexicographic (distance, id) sort."""
    b = base.astype(np.float64)
    ids = np.arange(base.shape[0]) if passing is None else np.nonzero(passing)[0]
    out_d = np.full((queries.shape[0], k), np.inf)
    out_i = np.full((queries.shape[0], k), -1, dtype=np.int64)
    for q in range(queries.shape[0]):
        d = ((b[ids] - queries[q].astype(np.float64)) ** 2).sum(axis=1)
        order = np.lexsort((ids, d))[:k]
        out_d[q, : len(order)] = d[order]
        out_i[q, : len(order)] = ids[order]
    return out_d, out_i


def test_topk_bruteforce_matches_closed_form():
    rng = np.random.default_rng(3)
    base = rng.standard_normal((3000, 24)).astype(np.float32)
    queries = rng.standard_normal((9, 24)).astype(np.float32)
    for k, passing in ((1, None), (17, None), (64, (rng.random(3000) < 0.1).astype(np.uint8))):
        got_d, got_i = orc.topk_bruteforce(base, queries, k, passing, n_threads=3)
        want_d, want_i = _topk_numpy(base, queries, k, passing)
        assert np.array_equal(got_i, want_i)
        assert np.allclose(got_d, want_d, rtol=1e-12)


def test_topk_bruteforce_ties_padding_and_empty():
    rng = np.random.default_rng(4)
    uniq = rng.standard_normal((5, 8)).astype(np.float32)
    base = np.ascontiguousarray(np.repeat(uniq, 7, axis=0)[rng.permutation(35)])  # exact ties
    queries = np.ascontiguousarray(uniq[:2])
    got_d, got_i = orc.topk_bruteforce(base, queries, 12, None, n_threads=2)
    want_d, want_i = _topk_numpy(base, queries, 12, None)
    assert np.array_equal(got_i, want_i)  # ties: smaller id first
    assert np.all(got_d[:, :7] == 0.0)
    passing = np.zeros(35, np.uint8)
    passing[[3, 30]] = 1
    got_d, got_i = orc.topk_bruteforce(base, queries, 5, passing)
    assert np.all(got_i[:, 2:] == -1) and np.all(np.isinf(got_d[:, 2:]))
    assert sorted(got_i[0, :2].tolist()) == [3, 30]
    got_d, got_i = orc.topk_bruteforce(base, queries, 3, np.zeros(35, np.uint8))
    assert np.all(got_i == -1)

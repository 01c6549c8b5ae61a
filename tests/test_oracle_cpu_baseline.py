"""Pins the CPU baselines bench.py times (oracle/cpu_baseline.c), CPU only:
each threaded function against the single-threaded oracle on the same input."""
import numpy as np
import pytest

import orc
from helpers import assert_same


@pytest.mark.parametrize("threads", [1, 4])
@pytest.mark.parametrize("case", ["uniform_2^24", "sparse_2^30", "clustered_2^26", "odd_u"])
def test_cpu_upload_matches_oracle(case, threads):
    rng = np.random.default_rng(sum(map(ord, case)))
    if case == "uniform_2^24":
        U, ids = 1 << 24, rng.integers(0, 1 << 24, 400_000, dtype=np.uint64)
    elif case == "sparse_2^30":  # most keys absent: containers move to their ranks
        U, ids = 1 << 30, rng.integers(0, 1 << 30, 5000, dtype=np.uint64)
    elif case == "clustered_2^26":
        U = 1 << 26
        parts = [np.arange(s, s + int(rng.integers(1000, 65536))) for s in rng.integers(0, U - 70000, 30)]
        ids = np.concatenate(parts)
        rng.shuffle(ids)
    else:
        U, ids = 3 * 65536 + 77, rng.integers(0, 3 * 65536 + 77, 20_000, dtype=np.uint64)
    ids = ids.astype(np.uint32)
    t, got = orc.cpu_upload_ids(ids, U, threads)
    assert t > 0
    assert_same(got, orc.upload_from_ids(ids, U), strict=True, what=f"cpu upload {case}")


def test_cpu_upload_rejects_complement_inputs():
    ids = np.arange(0, 60000, dtype=np.uint32)
    with pytest.raises(RuntimeError):
        orc.cpu_upload_ids(ids, 100000, 2)


def _operands(rng, U):
    a = np.unique(rng.integers(0, U, U // 1000, dtype=np.uint64)).astype(np.uint32)  # arrays
    b = np.nonzero(rng.random(U) < 0.5)[0].astype(np.uint32)  # bitsets
    runs = [np.arange(s, s + int(rng.integers(1000, 65536))) for s in rng.integers(0, U - 70000, 20)]
    c = np.unique(np.concatenate(runs)).astype(np.uint32)
    A, B, C = orc.Lite.from_ids(a), orc.Lite.from_ids(b), orc.Lite.from_ids(c).run_optimize()
    return A, B, C


@pytest.mark.parametrize("threads,n_shards", [(1, 1), (3, 7)])
def test_cpu_setop_matches_rl_op(threads, n_shards):
    U = 24 * 65536
    A, B, C = _operands(np.random.default_rng(3), U)
    for x, y in ((A, B), (B, C), (C, A), (A, A)):
        xs, ys = x.shards(n_shards, U >> 16), y.shards(n_shards, U >> 16)
        for op in (orc.AND, orc.OR, orc.ANDNOT, orc.XOR):
            want = x.op(y, op)
            t, card, nc = orc.cpu_setop(xs, ys, op, threads)
            assert t > 0 and card == want.cardinality() and nc == want.n_containers()


@pytest.mark.parametrize("threads,n_shards", [(1, 1), (4, 5)])
def test_cpu_multi_and_matches_chain(threads, n_shards):
    U = 16 * 65536
    A, B, C = _operands(np.random.default_rng(4), U)
    ins = [B, C, A, B]
    want = ins[0].op(ins[1], orc.AND).op(ins[2], orc.AND).op(ins[3], orc.AND)
    t, card, nc = orc.cpu_multi_and([x.shards(n_shards, U >> 16) for x in ins], threads)
    assert card == want.cardinality() and nc == want.n_containers()


@pytest.mark.parametrize("threads", [1, 5])
def test_cpu_contains_matches_rl(threads):
    U = 8 * 65536
    A, B, C = _operands(np.random.default_rng(5), U)
    q = np.random.default_rng(6).integers(0, 2 * U, 100_001, dtype=np.uint64).astype(np.uint32)
    for x in (A, B, C):
        t, got = orc.cpu_contains(x, q, threads)
        assert np.array_equal(got, x.contains_many(q))


def test_cpu_config0_matches_numpy():
    rng = np.random.default_rng(7)
    U = 1 << 20
    a = rng.integers(0, U, U // 100, dtype=np.uint64).astype(np.uint32)
    b = rng.integers(0, U, U // 10, dtype=np.uint64).astype(np.uint32)
    q = rng.integers(0, U, 50_000, dtype=np.uint64).astype(np.uint32)
    t, parts, cards, hits = orc.cpu_config0(a, b, q)
    sa, sb = set(a.tolist()), set(b.tolist())
    assert cards == [len(sa & sb), len(sa | sb), len(sa - sb), len(sa ^ sb)]
    assert hits == int(np.isin(q, a).sum())
    assert abs(sum(parts) - t) < 1e-6


@pytest.mark.parametrize("threads", [1, 3])
@pytest.mark.parametrize("filtered", [False, True])
def test_cpu_topk_fp32_matches_fp64(threads, filtered):
    rng = np.random.default_rng(8)
    n, d, nq, k = 3000, 40, 13, 10
    base = rng.standard_normal((n, d)).astype(np.float32)
    base[100] = base[7]  # an exact tie: the smaller id first
    queries = rng.standard_normal((nq, d)).astype(np.float32)
    queries[3] = base[7]
    passing = (rng.random(n) < 0.3).astype(np.uint8) if filtered else None
    if filtered:
        passing[[7, 100]] = 1
    t, dist, ids = orc.cpu_topk_fp32(base, queries, k, passing, threads)
    wd, wi = orc.topk_bruteforce(base, queries, k, passing)
    assert np.all(np.diff(dist, axis=1) >= 0)
    for i in range(nq):
        assert np.allclose(dist[i], wd[i], rtol=1e-4, atol=1e-6)
        kth = wd[i, -1]
        # identical id sets except ids tied with the k-th distance
        diff = set(ids[i].tolist()) ^ set(wi[i].tolist())
        for x in diff:
            dx = float(((base[x].astype(np.float64) - queries[i]) ** 2).sum())
            assert abs(dx - kth) <= 1e-4 * max(kth, 1e-12)
    assert ids[3, 0] == 7 and ids[3, 1] == 100  # the tie, smaller id first


def test_cpu_topk_fp32_fewer_rows_than_k():
    rng = np.random.default_rng(9)
    base = rng.standard_normal((50, 16)).astype(np.float32)
    q = rng.standard_normal((2, 16)).astype(np.float32)
    passing = np.zeros(50, np.uint8)
    passing[[3, 9, 44]] = 1
    t, dist, ids = orc.cpu_topk_fp32(base, q, 5, passing, 2)
    assert np.all(ids[:, 3:] == -1) and np.all(np.isinf(dist[:, 3:]))
    assert set(ids[0, :3].tolist()) == {3, 9, 44}

"""Pins roaring-lite (the CRoaring stand-in) against numpy brute force (CPU only)."""
import numpy as np
import pytest

import orc
from helpers import flat_from_ids, ids_from_flat


def _rand_set(rng, U, kind):
    if kind == "uniform":
        return np.unique(rng.integers(0, U, U // 20, dtype=np.uint32))
    if kind == "dense":
        return np.nonzero(rng.random(U) < 0.7)[0].astype(np.uint32)
    if kind == "runs":
        out = []
        for _ in range(8):
            s = int(rng.integers(0, U - 70000))
            out.append(np.arange(s, s + int(rng.integers(1000, 65536)), dtype=np.uint32))
        return np.unique(np.concatenate(out))
    if kind == "full":  # full containers and the 65535/65536 boundary
        return np.concatenate([np.arange(65536, 2 * 65536, dtype=np.uint32), np.array([65535, 3 * 65536], np.uint32)])
    return np.zeros(0, dtype=np.uint32)


KINDS = ["uniform", "dense", "runs", "full", "empty"]


@pytest.mark.parametrize("ka", KINDS)
@pytest.mark.parametrize("kb", KINDS)
def test_lite_ops_bruteforce(ka, kb):
    U = 5 * 65536
    rng = np.random.default_rng(sum(map(ord, ka + kb)))
    a, b = _rand_set(rng, U, ka), _rand_set(rng, U, kb)
    A, B = orc.Lite.from_ids(a), orc.Lite.from_ids(b)
    if ka == "runs":
        A.run_optimize()
    fa, fb = flat_from_ids(a, U), flat_from_ids(b, U)
    for op, want in ((orc.AND, fa & fb), (orc.OR, fa | fb), (orc.ANDNOT, fa & ~fb), (orc.XOR, fa ^ fb)):
        R = A.op(B, op)
        assert np.array_equal(flat_from_ids(R.to_ids(), U), want)
        assert R.cardinality() == int(np.unpackbits(want.view(np.uint8)).sum())
    q = rng.integers(0, U, 5000, dtype=np.uint32)
    assert np.array_equal(A.contains_many(q).astype(bool), np.isin(q, a))


def test_lite_flip():
    U = 200000
    rng = np.random.default_rng(3)
    a = np.unique(rng.integers(0, U, 50000, dtype=np.uint32))
    F = orc.Lite.from_ids(a).flip(0, U)
    assert np.array_equal(F.to_ids(), np.setdiff1d(np.arange(U, dtype=np.uint32), a))


def test_lite_container_types_and_run_optimize():
    # array iff card <= 4096; run iff 2 + 4*n_runs < current serialized size
    ids = np.concatenate([np.arange(4096, dtype=np.uint32),               # key 0: 4096 -> array; 1 run -> run
                          65536 + np.arange(4097, dtype=np.uint32) * 2,   # key 1: 4097 -> bitset; 4097 runs -> keep
                          2 * 65536 + np.arange(0, 20000, dtype=np.uint32)])  # key 2: bitset, 1 run -> run
    L = orc.Lite.from_sorted_ids(ids)
    assert [c[1] for c in L.containers()] == [orc.TC_ARRAY, orc.TC_BITSET, orc.TC_BITSET]
    L.run_optimize()
    conts = L.containers()
    assert [c[1] for c in conts] == [orc.TC_RUN, orc.TC_BITSET, orc.TC_RUN]
    assert conts[0][2] == 1 and list(conts[0][3]) == [0, 4095]
    assert np.array_equal(L.to_ids(), ids)
    # run count rule computed independently: array of 3 isolated values stays array
    L2 = orc.Lite.from_sorted_ids(np.array([1, 5, 9], dtype=np.uint32)).run_optimize()
    assert L2.containers()[0][1] == orc.TC_ARRAY
    # 2 runs of 3 values: run size 2+8=10 < array 2+12=14 -> run
    L3 = orc.Lite.from_sorted_ids(np.array([1, 2, 3, 7, 8, 9], dtype=np.uint32)).run_optimize()
    assert L3.containers()[0][1] == orc.TC_RUN


def test_upload_packed_counts():  # test/test_upload.cu:48-82 and test/test_promote.cu:41-165
    ids = np.concatenate([np.arange(100, dtype=np.uint32) * 10, 65536 + np.arange(50000, dtype=np.uint32),
                          131072 + np.arange(10000, dtype=np.uint32)])
    L = orc.Lite.from_sorted_ids(ids).run_optimize()
    r = orc.upload_packed(L)
    assert r.n_containers == 3 and r.n_array_containers + r.n_run_containers > 0
    assert np.array_equal(orc.decompress(r), flat_from_ids(ids, r.universe_size))
    p = orc.upload_packed(L, None, orc.PROMOTE_ALL)
    assert p.n_bitmap_containers == 3 and p.n_array_containers == 0 and p.n_run_containers == 0
    assert np.array_equal(orc.decompress(p), orc.decompress(r))
    full3 = orc.upload_packed(orc.Lite.from_sorted_ids(np.arange(3 * 65536, dtype=np.uint32)))
    assert full3.n_bitmap_containers == 3 and list(full3.cards) == [0, 0, 0]
    one = orc.upload_packed(orc.Lite.from_sorted_ids(np.array([7], np.uint32)))
    assert one.n_array_containers == 1 and one.universe_size == 65536
    top = orc.upload_packed(orc.Lite.from_sorted_ids(np.array([0xFFFFFFFF], np.uint32)))
    assert top.universe_size == 0  # (0xFFFF + 1) << 16 wraps (src/upload.cpp:96-100)
    empty = orc.upload_packed(orc.Lite.from_sorted_ids(np.zeros(0, np.uint32)), 1000)
    assert empty.n_containers == 0 and empty.universe_size == 1000


def test_upload_packed_auto_guard():  # src/upload.cpp:112-118
    # U = 2^26 -> AUTO says ALL, but 600 containers * 16 KiB >= 8 MiB flat -> guard keeps types
    U = 1 << 26
    rng = np.random.default_rng(0)
    ids = np.unique(rng.integers(0, U, 600 * 10, dtype=np.uint32))
    L = orc.Lite.from_sorted_ids(ids)
    r = orc.upload_packed(L, U)
    assert r.n_containers > 512 and r.n_array_containers == r.n_containers
    few = orc.Lite.from_sorted_ids(np.array([1, 2, 3, 1 << 25], dtype=np.uint32))
    r = orc.upload_packed(few, U)
    assert r.n_bitmap_containers == 2  # promoted: 2 * 16 KiB < 8 MiB
    r = orc.upload_packed(L, U, orc.PROMOTE_ALL)  # explicit ALL ignores the guard
    assert r.n_bitmap_containers == r.n_containers


@pytest.mark.parametrize("kind", KINDS)
def test_lite_from_words_matches_from_ids(kind):
    U = 5 * 65536 + 100
    rng = np.random.default_rng(11)
    ids = _rand_set(rng, U, kind)
    w = flat_from_ids(ids, U)
    a, b = orc.Lite.from_words(w), orc.Lite.from_ids(ids)
    ca, cb = a.containers(), b.containers()
    assert len(ca) == len(cb)
    for x, y in zip(ca, cb):
        assert x[:3] == y[:3] and np.array_equal(x[3], y[3])

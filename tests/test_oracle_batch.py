"""Pins the batch oracle (oracle/batch.py) on the CPU.

The first tests restate the reference's v2 test (v2/test/test_basic.cu:58-430)
with roaring-lite as the CRoaring stand-in: the same mixed inputs, probe set
and assertions.  The rest compare with flat-bitset brute force on random
batches.
"""
import numpy as np
import pytest

import batch as ob
import orc


def mixed_ids(variant: int) -> np.ndarray:
    """build_mixed_bitmap (v2/test/test_basic.cu:61-92) as a sorted id list."""
    stride = 13 + variant
    parts = [np.array([(i * stride) % 65536 for i in range(200)])]
    parts.append(np.arange(65536 + variant * 1000, 65536 + 60000))
    parts.append(np.arange(131072 + variant * 100, 131072 + 50000))
    if variant >= 2:
        parts.append(196608 + 7 * np.arange(50))
    return np.unique(np.concatenate(parts)).astype(np.uint32)


def mixed_lite(variant: int):
    return orc.Lite.from_sorted_ids(mixed_ids(variant)).run_optimize()


PROBES = np.arange(0, 280000, 37, dtype=np.uint32)  # build_probe_set (:94-99)


def test_n1_smoke():  # run_n1_smoke (:143-206)
    lite = mixed_lite(0)
    B = ob.upload_batch([lite.containers()])
    assert B.n_bitmaps == 1 and int(B.host_total_cardinalities[0]) == lite.cardinality()
    want = lite.contains_many(PROBES).astype(np.uint8)
    assert np.array_equal(ob.contains(B, 0, PROBES), want)
    assert np.array_equal(ob.view_contains(B, 0, PROBES), want)
    P = ob.promote_batch(B)
    assert P.n_bitmap_containers_total == P.total_containers
    assert np.array_equal(ob.contains(P, 0, PROBES), want)
    S = ob.multi_and(P, [0])
    assert int(S.host_total_cardinalities[0]) == int(P.host_total_cardinalities[0])
    assert np.array_equal(ob.contains(S, 0, PROBES), want)


def test_n4_full():  # run_n4_full (:208-420)
    lites = [mixed_lite(v) for v in range(4)]
    B = ob.upload_batch([l.containers() for l in lites])
    assert B.n_bitmaps == 4 and int(B.host_container_starts[4]) == B.total_containers
    for b, l in enumerate(lites):
        assert int(B.host_total_cardinalities[b]) == l.cardinality()
        assert int(B.host_container_starts[b + 1] - B.host_container_starts[b]) == l.n_containers()
        want = l.contains_many(PROBES).astype(np.uint8)
        assert np.array_equal(ob.contains(B, b, PROBES), want)
        assert np.array_equal(ob.view_contains(B, b, PROBES), want)
    P = ob.promote_batch(B)
    assert (P.n_bitmaps, P.total_containers, P.n_bitmap_containers_total) == (4, B.total_containers, B.total_containers)
    assert P.array_pool_bytes == 0 and P.run_pool_bytes == 0
    assert np.array_equal(P.host_total_cardinalities, B.host_total_cardinalities)
    for b, l in enumerate(lites):
        assert np.array_equal(ob.contains(P, b, PROBES), l.contains_many(PROBES).astype(np.uint8))
    for idx in ([0, 1, 2], [2, 3]):
        exp = lites[idx[0]]
        for j in idx[1:]:
            exp = exp.op(lites[j], orc.AND)
        R = ob.multi_and(P, idx)
        assert int(R.host_total_cardinalities[0]) == exp.cardinality()
        assert np.array_equal(ob.contains(R, 0, PROBES), exp.contains_many(PROBES).astype(np.uint8))
    with pytest.raises(ValueError):
        ob.multi_and(B, [0, 1])  # the raw batch still holds array / run containers
    words_each = (int(B.host_universe_sizes.max()) + 63) // 64
    flat = ob.decompress_batch(B, words_each)
    for b, l in enumerate(lites):
        slot = flat[b * words_each:(b + 1) * words_each]
        keep = PROBES[PROBES < B.host_universe_sizes[b]]
        bits = (slot[keep // 64] >> (keep % 64).astype(np.uint64)) & np.uint64(1)
        assert np.array_equal(bits.astype(np.uint8), l.contains_many(keep).astype(np.uint8))


def _random_lites(rng, n):
    out, sets = [], []
    for _ in range(n):
        parts = []
        for key in rng.choice(12, int(rng.integers(0, 8)), replace=False):
            base = int(key) * 65536
            kind = int(rng.integers(0, 4))
            if kind == 0:
                parts.append(base + np.unique(rng.integers(0, 65536, int(rng.integers(1, 3000)))))
            elif kind == 1:
                parts.append(base + np.nonzero(rng.random(65536) < rng.uniform(0.1, 0.9))[0])
            elif kind == 2:
                s = int(rng.integers(0, 50000))
                parts.append(base + np.arange(s, s + int(rng.integers(1, 15000))))
            else:
                parts.append(base + np.arange(65536))
        ids = np.unique(np.concatenate(parts)).astype(np.uint32) if parts else np.zeros(0, np.uint32)
        out.append(orc.Lite.from_sorted_ids(ids).run_optimize())
        sets.append(ids)
    return out, sets


@pytest.mark.parametrize("seed", range(5))
def test_random_batches_against_flat_sets(seed):
    rng = np.random.default_rng(seed)
    lites, sets = _random_lites(rng, 6)
    B = ob.upload_batch([l.containers() for l in lites])
    words_each = 12 * 1024
    flat = ob.decompress_batch(B, words_each)
    for b, ids in enumerate(sets):
        want = np.zeros(words_each * 64, bool)
        want[ids] = True
        got = np.unpackbits(flat[b * words_each:(b + 1) * words_each].view(np.uint8), bitorder="little")
        assert np.array_equal(got.astype(bool), want)
        q = rng.integers(0, 14 * 65536, 3000).astype(np.uint32)
        truth = np.isin(q, ids).astype(np.uint8)
        assert np.array_equal(ob.contains(B, b, q), truth)
        assert np.array_equal(ob.view_contains(B, b, q), truth)
    P = ob.promote_batch(B)
    for b, ids in enumerate(sets):
        for c in range(int(P.container_starts[b]), int(P.container_starts[b + 1])):
            key = int(P.keys[c])
            n_in = int(np.count_nonzero((ids >> 16) == key))
            assert int(P.cards[c]) == (0 if n_in == 65536 else n_in)
    idx = [int(i) for i in rng.choice(6, 3, replace=False)]
    R = ob.multi_and(P, idx)
    inter = sets[idx[0]]
    for j in idx[1:]:
        inter = np.intersect1d(inter, sets[j])
    assert int(R.host_total_cardinalities[0]) == inter.size
    q = np.concatenate([inter, rng.integers(0, 12 * 65536, 2000).astype(np.uint32)])
    assert np.array_equal(ob.contains(R, 0, q), np.isin(q, inter).astype(np.uint8))
    # zero-card common containers are kept; keys are the anchor keys present everywhere
    common = set(int(k) for k in P.keys[P.container_starts[idx[0]]:P.container_starts[idx[0] + 1]])
    for j in idx[1:]:
        common &= set(int(k) for k in P.keys[P.container_starts[j]:P.container_starts[j + 1]])
    if any(P.container_starts[j + 1] == P.container_starts[j] for j in idx):
        common = set()
    assert sorted(common) == [int(k) for k in R.keys]


def test_decompress_or_semantics_and_bounds():
    lites = [mixed_lite(2)]
    B = ob.upload_batch([l.containers() for l in lites])
    words_each = (int(B.host_universe_sizes[0]) + 63) // 64
    prior = np.full(words_each, np.uint64(0x8000000000000001), np.uint64)
    out = ob.decompress_batch(B, words_each, prior)
    # key 0 is an ARRAY: OR-ed into the prior words; keys 1 and 2 are RUN: OR-ed too
    img0 = ob.container_image(B, 0)
    assert np.array_equal(out[:1024], img0 | prior[:1024])
    with pytest.raises(ValueError):
        ob.decompress_batch(B, words_each - 1)

"""GPU parity: the HIP library through the C-ABI vs the CPU oracle, bit-exact.

Every case prints what it runs before touching the GPU.  Sizes are chosen so
the oracle finishes in seconds; full-size configurations are covered by the
property tests in test_gpu_scale.py.
"""
import numpy as np
import pytest

import orc
from helpers import assert_packed_offsets, assert_same, flat_from_ids, mt_bernoulli, mt_mod_filter, words_mask, auto_l2

pytestmark = pytest.mark.gpu


def _say(*a):
    print("CASE", *a, flush=True)


def _torch():
    import torch
    return torch


def _dev_u32(a):
    torch = _torch()
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).cuda()


# ---- upload_from_ids --------------------------------------------------------
ID_CASES = [
    # (n, universe, threshold, seed)
    (1, 1000, orc.PROMOTE_KEEP_DEFAULT, 1),
    (8, 200000, orc.PROMOTE_KEEP_DEFAULT, 2),
    (500, 5 * 65536, orc.PROMOTE_ALL, 3),
    (1000, 1 << 20, orc.PROMOTE_AUTO, 4),
    (1024, 70000, 100, 5),
    (1025, 70000, orc.PROMOTE_AUTO, 6),
    (5000, 1 << 22, orc.PROMOTE_AUTO, 7),
    (200000, 1 << 24, orc.PROMOTE_KEEP_DEFAULT, 8),
    (300000, 1 << 30, orc.PROMOTE_AUTO, 9),
    (50000, 0xFFFFFFFF, orc.PROMOTE_AUTO, 10),
    # around the GPU path's 24576-id tiles and its blocks of 8 tiles
    (24576, 1 << 26, orc.PROMOTE_AUTO, 11),
    (24577, 1 << 26, orc.PROMOTE_AUTO, 12),
    (24576 * 2 + 5, 1 << 24, orc.PROMOTE_AUTO, 13),
    (24576 * 8 + 1, 1 << 28, orc.PROMOTE_AUTO, 14),
    (24576 * 9 - 1, 1 << 30, orc.PROMOTE_KEEP_DEFAULT, 15),
    # more than 1024 ids but fewer than keys: the metadata arrays hold n entries, not K
    (1025, 1 << 30, orc.PROMOTE_AUTO, 16),
    (2000, 1 << 30, orc.PROMOTE_AUTO, 17),
    (5000, 1 << 30, orc.PROMOTE_KEEP_DEFAULT, 18),
    (1025, 0xFFFFFFFF, orc.PROMOTE_AUTO, 19),
    (20000, 0xFFFFFFFF, orc.PROMOTE_AUTO, 20),
    (16383, 1 << 30, orc.PROMOTE_AUTO, 21),
    # 2048 and 3072 buckets: the tile sort's bucket scan spans two and three waves
    (60000, 1 << 31, orc.PROMOTE_AUTO, 22),
    (70000, 3 << 30, orc.PROMOTE_AUTO, 23),
]


@pytest.mark.parametrize("n,universe,thr,seed", ID_CASES)
def test_upload_from_ids_parity(gpu, n, universe, thr, seed):
    _say("upload_from_ids", n, universe, thr, seed)
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, universe, n, dtype=np.uint64).astype(np.uint32)
    if n > 10:
        ids[: n // 10] = ids[n // 10: 2 * (n // 10)]  # ~10% duplicates
    want = orc.upload_from_ids(ids, universe, thr, auto_l2(gpu))
    g = gpu.upload_from_ids(ids, universe, thr)
    got = gpu.download(g)
    assert_same(got, want, strict=True, what="upload_from_ids")
    gpu.free(g)
    g = gpu.upload_from_device_ids(_dev_u32(ids), universe, thr)
    assert_same(gpu.download(g), want, strict=True, what="upload_from_device_ids")
    gpu.free(g)


@pytest.mark.parametrize("case", ["small_negated", "absent_key", "large_gpu_path", "reversed_all", "half",
                                  "dense_clustered", "full_containers"])
def test_upload_from_ids_complement_cases(gpu, case):
    _say("upload_from_ids complement", case)
    if case == "small_negated":  # test/test_complement.cu:129-149
        ids, U = np.array([0, 1, 2, 3, 4, 5, 6, 8, 9], np.uint32), 10
    elif case == "absent_key":  # :151-182
        ids, U = mt_mod_filter(42, 200000, 10, keep_zero=False), 200000
    elif case == "large_gpu_path":  # :184-210
        ids, U = mt_mod_filter(123, 100000, 5, keep_zero=False), 100000
    elif case == "reversed_all":  # test/test_promote.cu:431-449
        ids, U = np.arange(999, -1, -1, dtype=np.uint32), 1000
    elif case == "half":  # :227-237 (not negated)
        ids, U = np.arange(50, dtype=np.uint32), 100
    elif case == "dense_clustered":
        ids, U = np.concatenate([np.arange(0, 300000), np.arange(400000, 1000000)]).astype(np.uint32), 1048576
    else:
        ids, U = np.arange(3 * 65536 + 5, dtype=np.uint32), 4 * 65536 + 17
    want = orc.upload_from_ids(ids, U)
    g = gpu.upload_from_ids(ids, U)
    assert_same(gpu.download(g), want, strict=True, what=case)
    gpu.free(g)


@pytest.mark.parametrize("order", ["sorted", "reverse", "clustered_shuffled", "one_bucket", "skewed"])
def test_upload_from_ids_input_orders(gpu, order):
    """Inputs whose waves fall in one bucket (sorted runs), runs far longer than a
    tile's typical bucket run, partial tile blocks and a skewed key distribution."""
    _say("upload_from_ids order", order)
    rng = np.random.default_rng(77)
    U = 1 << 26
    if order == "sorted":
        ids = np.sort(rng.integers(0, U, 3_000_000, dtype=np.uint64)).astype(np.uint32)
    elif order == "reverse":
        ids = np.arange(U - 1, U - 2_500_001, -1, dtype=np.int64).astype(np.uint32)
    elif order == "clustered_shuffled":  # runs of length U[1000, 65536), then shuffled (BASELINE clustered variant)
        parts, total = [], 0
        while total < 2_000_000:
            ln = int(rng.integers(1000, 65536))
            st = int(rng.integers(0, U - ln))
            parts.append(np.arange(st, st + ln, dtype=np.uint32))
            total += ln
        ids = np.concatenate(parts)
        ids = np.concatenate([ids, ids[rng.integers(0, ids.size, ids.size // 10)]])
        ids = ids[rng.permutation(ids.size)]
    elif order == "one_bucket":  # every id in one 16-key bucket, more than one tile block
        ids = rng.integers(5 << 20, 6 << 20, 300_000, dtype=np.uint64).astype(np.uint32)
    else:  # half the ids in one key, the rest uniform
        ids = np.concatenate([rng.integers(7 << 16, 8 << 16, 600_000, dtype=np.uint64),
                              rng.integers(0, U, 600_000, dtype=np.uint64)]).astype(np.uint32)
        ids = ids[rng.permutation(ids.size)]
    want = orc.upload_from_ids(ids, U)
    g = gpu.upload_from_device_ids(_dev_u32(ids), U)
    assert_same(gpu.download(g), want, strict=True, what=order)
    gpu.free(g)


def test_upload_from_ids_rejects_out_of_universe_keys(gpu):
    _say("upload_from_ids invalid")
    ids = np.arange(2000, dtype=np.uint32) + (5 << 16)
    with pytest.raises(gpu.CrError) as e:
        gpu.upload_from_ids(ids, 65536)
    assert e.value.code == 2


@pytest.mark.parametrize("bad_key", [25, 40, 0xFFFF])
def test_upload_from_ids_rejects_keys_past_the_last_bucket(gpu, bad_key):
    """20 keys = 2 buckets of 16: key 25 lies in the last bucket but past max_key,
    keys 40 and 0xFFFF lie past the last bucket.  One such id fails the call."""
    _say("upload_from_ids invalid key", bad_key)
    ids = np.arange(50000, dtype=np.uint32) * 7 % (20 * 65536)
    ids[12345] = (bad_key << 16) | 7
    with pytest.raises(gpu.CrError) as e:
        gpu.upload_from_device_ids(_dev_u32(ids), 20 * 65536)
    assert e.value.code == 2


@pytest.mark.parametrize("n", [16384 * 3 + 5, 24576 * 3 + 5, 24576 * 9])
def test_upload_from_ids_unaligned_pointer(gpu, n):
    """A device pointer 4 bytes past a 16-byte boundary takes the scalar load
    path, with and without a partial last tile."""
    _say("upload_from_ids unaligned", n)
    rng = np.random.default_rng(n)
    U = 1 << 24
    ids = rng.integers(0, U, n + 1, dtype=np.uint64).astype(np.uint32)
    d = _dev_u32(ids)
    view = d[1:]
    assert view.data_ptr() % 16 == 4
    want = orc.upload_from_ids(ids[1:], U)
    g = gpu.upload_from_device_ids(view, U)
    assert_same(gpu.download(g), want, strict=True, what="unaligned")
    gpu.free(g)


@pytest.mark.parametrize("offset", [1, 3])
def test_contains_partitioned_unaligned_and_partial_tiles(gpu, offset):
    """Mode 4 with a query pointer off a 16-byte boundary (the tile sort's scalar
    loads and the permutation in that order), an unaligned output, and a tile
    count that is not a multiple of the tile blocks."""
    _say("contains partitioned unaligned", offset)
    torch = _torch()
    rng = np.random.default_rng(90 + offset)
    U = 1 << 26
    ids = np.nonzero(rng.random(U) < 0.05)[0].astype(np.uint32)
    g, want = gpu.upload_from_ids(ids, U), orc.upload_from_ids(ids, U)
    q = rng.integers(0, 2 * U, 24576 * 9 + 77, dtype=np.uint64).astype(np.uint32)
    dq = _dev_u32(np.concatenate([np.zeros(offset, np.uint32), q]))[offset:]
    out = torch.empty(q.size + offset, dtype=torch.int32, device="cuda")[offset:]
    assert dq.data_ptr() % 16 != 0 and out.data_ptr() % 16 != 0
    gpu.contains_batch(g, dq, out, 4)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), orc.contains_many(want, q))
    gpu.free(g)


@pytest.mark.parametrize("universe", [1 << 31, 3 << 30, 0xFFFFFFFF])
def test_contains_partitioned_many_buckets(gpu, universe):
    """Mode 4 on bitmaps whose keys reach 2^31, 3 * 2^30 and 2^32: 2048 to 4096
    buckets of 16 keys, so the tile sort's bucket scan spans two to four waves
    and its run table is written straight to memory; queries past the last key
    fall in the sentinel bucket (none at 2^32)."""
    _say("contains partitioned many buckets", universe)
    torch = _torch()
    rng = np.random.default_rng(95 + (universe >> 30))
    ids = rng.integers(0, universe, 400000, dtype=np.uint64).astype(np.uint32)
    g, want = gpu.upload_from_ids(ids, universe), orc.upload_from_ids(ids, universe)
    q = np.concatenate([ids[:100000], rng.integers(0, 1 << 32, 24576 * 5 + 11, dtype=np.uint64).astype(np.uint32)])
    out = torch.empty(q.size, dtype=torch.int32, device="cuda")
    gpu.contains_batch(g, _dev_u32(q), out, 4)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), orc.contains_many(want, q))
    gpu.free(g)


@pytest.mark.parametrize("density", [0.05, 0.6])
def test_contains_partitioned_sentinel_tiles(gpu, density):
    """Mode 4 with whole tiles of queries past the bitmap's last bucket (the tile
    sort's sentinel bucket): such a tile has no field of a real bucket to write
    out, and its answers are all `negated` (a density above 1/2 uploads as a
    negated complement); a mixed tile, an ordinary one and a partial one follow."""
    _say("contains partitioned sentinel tiles", density)
    torch = _torch()
    rng = np.random.default_rng(97)
    U = 1 << 24
    ids = np.nonzero(rng.random(U) < density)[0].astype(np.uint32)
    g, want = gpu.upload_from_ids(ids, U), orc.upload_from_ids(ids, U)
    assert bool(g.negated) == (density > 0.5)
    q = np.concatenate([rng.integers(1 << 28, 1 << 32, 24576 * 2, dtype=np.uint64),
                        rng.integers(0, 1 << 32, 24576, dtype=np.uint64),
                        rng.integers(0, U, 24576 + 5, dtype=np.uint64)]).astype(np.uint32)
    out = torch.empty(q.size, dtype=torch.int32, device="cuda")
    gpu.contains_batch(g, _dev_u32(q), out, 4)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint32)
    assert np.array_equal(got, orc.contains_many(want, q))
    assert np.all(got[:24576 * 2] == (1 if g.negated else 0))
    gpu.free(g)


def _skewed_ids(case, rng):
    """Inputs whose tiles each fall in a few key buckets (16 keys a bucket):
    long runs per (bucket, tile), shared by the whole build workgroup.
    "overflow" gives the single bucket of U = 2^20 more such tiles (2054) than
    the workgroup's queue holds (2048); the rest are finished by their wave.
    "heavy" puts half of 3M ids over 2^30 into four buckets, which the
    persistent build takes first among its ticketed buckets."""
    if case == "sorted":
        U = 1 << 26
        return U, np.sort(rng.integers(0, U, 24576 * 20 + 77, dtype=np.uint64)).astype(np.uint32)
    if case == "clustered":  # groups of 4096 sorted ids in random 65536-aligned windows
        U = 1 << 28
        win = rng.integers(0, U >> 16, 150, dtype=np.uint64)
        off = np.sort(rng.integers(0, 65536, (150, 4096), dtype=np.uint64), axis=1)
        return U, ((win[:, None] << 16) + off).reshape(-1).astype(np.uint32)
    if case == "heavy":  # a few buckets hold half the ids: the build's ordered tickets carry them
        U = 1 << 30
        uni = rng.integers(0, U, 1_500_000, dtype=np.uint64)
        # buckets 356, 704 and 1023 sit past their XCD range's static first round
        # (32 of 128 buckets at 2^30), bucket 131 inside it
        heavy = [(b << 20) + rng.integers(0, 1 << 20, 375_000, dtype=np.uint64) for b in (131, 356, 704, 1023)]
        ids = np.concatenate([uni] + heavy)
        return U, ids[rng.permutation(ids.size)].astype(np.uint32)
    U = 1 << 20
    allowed = np.nonzero(rng.random(U) < 0.9)[0].astype(np.uint32)
    return U, allowed[rng.integers(0, allowed.size, 24576 * 2054 + 5)]


@pytest.mark.parametrize("case", ["sorted", "clustered", "overflow", "heavy"])
def test_upload_and_partitioned_skewed(gpu, case):
    """upload_from_ids and mode 4 on inputs whose tiles hit few buckets: the
    walk's queued long runs, and its in-wave path once the queue is full."""
    _say("skewed ids", case)
    torch = _torch()
    rng = np.random.default_rng({"sorted": 70, "clustered": 71, "overflow": 72, "heavy": 73}[case])
    U, ids = _skewed_ids(case, rng)
    want = orc.upload_from_ids(ids, U, orc.PROMOTE_AUTO, auto_l2(gpu))
    dq = _dev_u32(ids)
    g = gpu.upload_from_device_ids(dq, U)
    assert_same(gpu.download(g), want, strict=True, what=f"upload {case}")
    # the same skew as queries: every id is a member; shifted ones mostly not
    flat = np.zeros(U + 1, np.uint8)
    flat[ids] = 1
    out = torch.empty(ids.size, dtype=torch.int32, device="cuda")
    for shift in (0, 1):
        q = dq if shift == 0 else _dev_u32((ids + 1) % U)
        gpu.contains_batch(g, q, out, 4)
        torch.cuda.synchronize()
        want_q = flat[(ids.astype(np.int64) + shift) % U].astype(np.uint32)
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want_q), (case, shift)
    gpu.free(g)


# ---- PROMOTE_AUTO on gfx950 ----------------------------------------------------
def test_resolve_auto_threshold_gfx950(gpu):
    """The re-derived rule (32 ceil(U/8) > one XCD's L2) keeps the reference's five
    pinned verdicts (test/test_promote.cu:257-381) and, at MI355X's 4 MiB per-XCD
    L2, promotes from U > 2^20, where the reference's rule keeps 2^21 .. 2^24
    compressed."""
    _say("resolve_auto_threshold")
    keep, all_ = orc.PROMOTE_KEEP_DEFAULT, orc.PROMOTE_ALL
    for u, want in ((1_000_000, keep), (1_000_000_000, all_), (100_000, keep), (1 << 30, all_), (10_000, keep),
                    (0, keep)):
        assert gpu.resolve_auto_threshold(u) == want, u
    if gpu.device_l2_bytes() == 4 << 20:
        assert gpu.resolve_auto_threshold(1 << 20) == keep
        assert gpu.resolve_auto_threshold((1 << 20) + 8) == all_
        for lg in (21, 22, 24):
            assert gpu.resolve_auto_threshold(1 << lg) == all_
            assert orc.resolve_auto_threshold(1 << lg, gpu.device_l2_bytes()) == keep  # the reference's rule


@pytest.mark.parametrize("n_keys", [8191, 8192])
def test_upload_auto_footprint_guard(gpu, n_keys):
    """The footprint term of PROMOTE_AUTO: upload() promotes under AUTO only while
    n_containers x 8 KiB x 2 < ceil(U/8) (src/upload.cpp:106-118), so at U = 2^30
    8191 sparse containers become bitmaps (64 MiB) and 8192 stay arrays (the
    promoted layout would be as large as the flat bitset).  promote_auto has no
    such guard (src/promote.cu:369-385): it promotes the 8192 arrays (and copies
    the 8191 bitmaps)."""
    _say("AUTO footprint guard", n_keys)
    U = 1 << 30
    keys = np.arange(n_keys, dtype=np.uint64) * 2  # every other key, 3 values each
    ids = np.sort(((keys << np.uint64(16))[:, None] + np.array([5, 700, 40000], dtype=np.uint64)).ravel())
    lite = orc.Lite.from_sorted_ids(ids.astype(np.uint32))
    want = orc.upload_packed(lite, U, orc.PROMOTE_AUTO, auto_l2(gpu))
    g = gpu.upload_containers(lite.containers(), U, False, lite.cardinality(), orc.PROMOTE_AUTO)
    assert_same(gpu.download(g), want, strict=True, what=f"AUTO guard {n_keys}")
    if gpu.resolve_auto_threshold(U) == orc.PROMOTE_ALL:
        assert (g.n_bitmap_containers, g.n_array_containers) == ((n_keys, 0) if n_keys < 8192 else (0, n_keys))
    p = gpu.promote_auto(g)
    gpu.synchronize()
    assert_same(gpu.download(p), orc.promote_auto(want, auto_l2(gpu)), strict=True, what=f"promote_auto {n_keys}")
    if gpu.resolve_auto_threshold(U) == orc.PROMOTE_ALL:
        assert p.n_bitmap_containers == n_keys  # 8191: already bitmaps (a copy); 8192: promoted
    gpu.free(p)
    gpu.free(g)


# ---- bitset uploads ----------------------------------------------------------
BITSET_CASES = [(100000, 0.1, 1), (100000, 0.9, 2), (200000, 1 / 3, 3), (5 * 65536 + 123, 0.001, 4),
                (5 * 65536 + 123, 0.95, 5), (1 << 22, 0.5, 6), (1 << 22, 0.55, 7), (64, 1.0, 8), (96, 0.0, 9)]


@pytest.mark.parametrize("invert", [False, True])
def test_upload_from_bitset_past_16_rounds(gpu, invert):
    """A universe just past 2^30: 16390 chunks, 17 rounds of the plan's 1024
    (the last partial), so its counts come in two passes of 16 rounds; sparse,
    and inverted (stored as the complement, from the inverted counts)."""
    _say("upload_from_bitset past 16 rounds", invert)
    U = (1 << 30) + 5 * 65536 + 123
    rng = np.random.default_rng(31 + int(invert))
    ids = np.unique(np.concatenate([rng.integers(0, U, 20000, dtype=np.uint64),
                                    U - 1 - 7 * np.arange(3000, dtype=np.uint64)])).astype(np.uint32)
    words = np.zeros((U + 31) // 32, np.uint32)  # built directly: no 2^30-entry bool array
    np.bitwise_or.at(words, (ids >> 5).astype(np.int64), np.left_shift(np.uint32(1), ids & np.uint32(31)))
    if invert:
        words = ~words
        words[-1] &= np.uint32((1 << (U % 32)) - 1)  # no bits past the universe
    want = orc.upload_from_bitset(words, U)
    g = gpu.upload_from_bitset(words, U)
    assert bool(g.negated) == invert
    assert_same(gpu.download(g), want, strict=True, what="bitset past 16 rounds")
    gpu.free(g)


@pytest.mark.parametrize("universe,density,seed", BITSET_CASES)
def test_upload_from_bitset_parity(gpu, universe, density, seed):
    _say("upload_from_bitset", universe, density, seed)
    rng = np.random.default_rng(seed)
    ids = np.nonzero(rng.random(universe) < density)[0].astype(np.uint32)
    words = flat_from_ids(ids, universe)
    want = orc.upload_from_bitset(words, universe)
    g = gpu.upload_from_bitset(words, universe)
    assert_same(gpu.download(g), want, strict=True, what="upload_from_bitset")
    gpu.free(g)
    g = gpu.upload_from_device_bitset(_dev_u32(words), universe)
    assert_same(gpu.download(g), want, strict=True, what="upload_from_device_bitset")
    gpu.free(g)


def test_upload_from_bitset_extra_words_and_tail(gpu):
    # n_words beyond ceil(U/32): inverted words past the tail stay all-ones (reference quirk)
    _say("upload_from_bitset extra words")
    U = 70000
    words = np.full(2200 + 2048, 0xFFFFFFFF, dtype=np.uint32)
    words[100] = 0
    want = orc.upload_from_bitset(words, U)
    g = gpu.upload_from_bitset(words, U)
    assert_same(gpu.download(g), want, strict=True, what="extra words")
    gpu.free(g)


# ---- packed upload ------------------------------------------------------------
def _lite_sets():
    rng = np.random.default_rng(11)
    U = 8 * 65536
    sparse = np.unique(rng.integers(0, U, 2000, dtype=np.uint32))
    dense = np.nonzero(rng.random(U) < 0.6)[0].astype(np.uint32)
    runs = np.unique(np.concatenate([np.arange(s, s + l) for s, l in ((1000, 5000), (70000, 65000), (300000, 9))]))
    mixed = np.unique(np.concatenate([sparse[:500], dense[dense < 2 * 65536], runs]).astype(np.uint32))
    return U, {"sparse": sparse, "dense": dense, "runs": runs.astype(np.uint32), "mixed": mixed}


@pytest.mark.parametrize("name", ["sparse", "dense", "runs", "mixed"])
@pytest.mark.parametrize("thr", [orc.PROMOTE_KEEP_DEFAULT, orc.PROMOTE_ALL, orc.PROMOTE_AUTO, 100])
@pytest.mark.parametrize("with_u", [False, True])
def test_upload_containers_parity(gpu, name, thr, with_u):
    _say("upload_containers", name, thr, with_u)
    U, sets = _lite_sets()
    lite = orc.Lite.from_sorted_ids(sets[name]).run_optimize()
    want = orc.upload_packed(lite, U if with_u else None, thr, auto_l2(gpu))
    if with_u and lite.cardinality() > U // 2:
        src, comp = lite.flip(0, U), True
    else:
        src, comp = lite, False
    g = gpu.upload_containers(src.containers(), U if with_u else 0, comp, lite.cardinality(), thr)
    got = gpu.download(g)
    assert_same(got, want, strict=True, what="upload_containers")
    assert_packed_offsets(got, what="upload_containers")
    gpu.free(g)


# ---- set operations -----------------------------------------------------------
def _build_operands(seed):
    """A mix of array / bitmap / run containers with shared and one-sided keys."""
    rng = np.random.default_rng(seed)
    U = 12 * 65536
    parts_a, parts_b = [], []
    for key in range(12):
        base = key * 65536
        kind_a, kind_b = rng.integers(0, 5, 2)
        for kind, parts in ((kind_a, parts_a), (kind_b, parts_b)):
            if kind == 0:
                continue  # key absent
            if kind == 1:
                parts.append(base + np.unique(rng.integers(0, 65536, int(rng.integers(1, 3000)))))
            elif kind == 2:
                parts.append(base + np.nonzero(rng.random(65536) < rng.uniform(0.1, 0.9))[0])
            elif kind == 3:
                s = int(rng.integers(0, 30000))
                parts.append(base + np.arange(s, s + int(rng.integers(100, 35000))))
            else:
                parts.append(base + np.arange(65536))  # full container
    a = np.unique(np.concatenate(parts_a)).astype(np.uint32) if parts_a else np.zeros(0, np.uint32)
    b = np.unique(np.concatenate(parts_b)).astype(np.uint32) if parts_b else np.zeros(0, np.uint32)
    la = orc.Lite.from_sorted_ids(a).run_optimize()
    lb = orc.Lite.from_sorted_ids(b).run_optimize()
    return U, la, lb


def _upload_pair(gpu, lite, U, thr, negate=False):
    if negate:
        comp = lite.flip(0, U)
        want = orc.upload_packed(comp, None, thr, auto_l2(gpu))
        want.negated, want.universe_size, want.total_cardinality, want._c = True, U, lite.cardinality(), None
        g = gpu.upload_containers(comp.containers(), 0, False, 0, thr)
        g.negated, g.universe_size, g.total_cardinality = True, U, lite.cardinality()
        return g, want
    want = orc.upload_packed(lite, None, thr, auto_l2(gpu))
    return gpu.upload_containers(lite.containers(), 0, False, 0, thr), want


@pytest.mark.parametrize("seed", [1, 2, 3, 4, 5, 6])
@pytest.mark.parametrize("op", [orc.AND, orc.OR, orc.ANDNOT, orc.XOR])
def test_set_operation_mixed_parity(gpu, seed, op):
    _say("set_operation mixed", seed, op)
    U, la, lb = _build_operands(seed)
    ga, oa = _upload_pair(gpu, la, U, orc.PROMOTE_KEEP_DEFAULT)
    gb, ob = _upload_pair(gpu, lb, U, orc.PROMOTE_KEEP_DEFAULT)
    want = orc.set_operation(oa, ob, op)
    g = gpu.set_operation(ga, gb, op)
    assert_same(gpu.download(g), want, strict=True, what=f"setop {op}")
    for x in (g, ga, gb):
        gpu.free(x)


@pytest.mark.parametrize("op", [orc.AND, orc.OR, orc.ANDNOT, orc.XOR])
@pytest.mark.parametrize("order", ["result_first", "result_second"])
def test_set_operation_on_a_result(gpu, op, order):
    """One operand is a set-operation result, which carries no key_index, the
    other an upload, which does: the plan finds the result's keys by searching
    them, the upload's through its key_index."""
    _say("set_operation on a result", op, order)
    U, la, lb = _build_operands(3)
    _, lc = _build_operands(4)[1:]
    ga, oa = _upload_pair(gpu, la, U, orc.PROMOTE_KEEP_DEFAULT)
    gb, ob = _upload_pair(gpu, lb, U, orc.PROMOTE_KEEP_DEFAULT)
    gc, oc = _upload_pair(gpu, lc, U, orc.PROMOTE_KEEP_DEFAULT)
    gr, orr = gpu.set_operation(ga, gb, orc.OR), orc.set_operation(oa, ob, orc.OR)
    assert not gr.key_index and gc.key_index
    x, ox, y, oy = (gr, orr, gc, oc) if order == "result_first" else (gc, oc, gr, orr)
    g = gpu.set_operation(x, y, op)
    assert_same(gpu.download(g), orc.set_operation(ox, oy, op), strict=True, what=f"setop on a result {op}")
    for h in (g, gr, ga, gb, gc):
        gpu.free(h)


@pytest.mark.parametrize("op", [orc.AND, orc.OR, orc.ANDNOT, orc.XOR])
@pytest.mark.parametrize("na", [False, True])
@pytest.mark.parametrize("nb", [False, True])
def test_set_operation_demorgan_parity(gpu, op, na, nb):  # test/test_complement.cu:367-462
    _say("set_operation demorgan", op, na, nb)
    U = 100000
    la = orc.Lite.from_sorted_ids(mt_bernoulli(42, 0.3, U))
    lb = orc.Lite.from_sorted_ids(mt_bernoulli(99, 0.4, U))
    ga, oa = _upload_pair(gpu, la, U, orc.PROMOTE_AUTO, negate=na)
    gb, ob = _upload_pair(gpu, lb, U, orc.PROMOTE_AUTO, negate=nb)
    want = orc.set_operation(oa, ob, op)
    g = gpu.set_operation(ga, gb, op)
    got = gpu.download(g)
    assert_same(got, want, strict=True, what="demorgan")
    logical = {orc.AND: np.intersect1d, orc.OR: np.union1d, orc.ANDNOT: np.setdiff1d,
               orc.XOR: np.setxor1d}[op](la.to_ids(), lb.to_ids())
    assert np.array_equal(words_mask(orc.decompress(got, (U + 31) // 32), U), words_mask(flat_from_ids(logical, U), U))
    for x in (g, ga, gb):
        gpu.free(x)


@pytest.mark.parametrize("op", [orc.AND, orc.OR, orc.ANDNOT, orc.XOR])
def test_set_operation_all_bitmap_large(gpu, op):
    _say("set_operation all-bitmap", op)
    U = 1 << 26
    rng = np.random.default_rng(77 + op)
    a = rng.integers(0, U, 3_000_000, dtype=np.uint32)
    b = rng.integers(0, U // 2, 2_000_000, dtype=np.uint32)
    oa, ob = orc.upload_from_ids(a, U), orc.upload_from_ids(b, U)
    ga, gb = gpu.upload_from_ids(a, U), gpu.upload_from_ids(b, U)
    want = orc.set_operation(oa, ob, op)
    g = gpu.set_operation(ga, gb, op)
    assert_same(gpu.download(g), want, strict=True, what="bb large")
    for x in (g, ga, gb):
        gpu.free(x)


@pytest.mark.parametrize("op", [orc.AND, orc.OR, orc.ANDNOT, orc.XOR])
def test_set_operation_understated_counts_fall_back(gpu, op):
    """Inputs whose type counts and pool sizes understate their containers (all
    zero: the struct claims to be all-bitmap with empty pools).  The one-sync
    path sizes its output from those counts; the plan kernel finds that the
    plan does not fit (or is not bitmap-only), nothing is written, and the call
    redoes the work on the exact two-pass path: the result is the oracle's."""
    _say("set_operation understated counts", op)
    U, la, lb = _build_operands(3)
    ga, oa = _upload_pair(gpu, la, U, orc.PROMOTE_KEEP_DEFAULT)
    gb, ob = _upload_pair(gpu, lb, U, orc.PROMOTE_KEEP_DEFAULT)
    assert ga.n_array_containers + ga.n_run_containers > 0
    want = orc.set_operation(oa, ob, op)
    bad = []
    for g in (ga, gb):
        x = gpu.GpuRoaring.from_buffer_copy(g)  # aliases g's device block; not freed itself
        x.n_bitmap_containers = x.n_array_containers = x.n_run_containers = 0
        x.array_pool_bytes = x.run_pool_bytes = 0
        bad.append(x)
    r = gpu.set_operation(bad[0], bad[1], op)
    assert_same(gpu.download(r), want, strict=True, what=f"understated counts {op}")
    for x in (r, ga, gb):
        gpu.free(x)


@pytest.mark.parametrize("op", [orc.AND, orc.OR, orc.ANDNOT, orc.XOR])
@pytest.mark.parametrize("case", ["random", "identical", "with_empty_results"])
def test_set_operation_dense_all_bitmap(gpu, op, case):
    """Two all-bitmap inputs with a container for every key of [0, max_key]: the
    plan-free path (pair i is key i).  Identical inputs drop every XOR and ANDNOT
    result; disjoint halves of each key drop AND results; full containers are
    stored with card 0 and dropped by AND."""
    _say("set_operation dense", op, case)
    rng = np.random.default_rng(5 + op)
    U = 40 * 65536
    a = np.nonzero(rng.random(U) < 0.3)[0].astype(np.uint32)
    if case == "random":
        b = np.nonzero(rng.random(U) < 0.6)[0].astype(np.uint32)
    elif case == "identical":
        b = a.copy()
    else:  # keys 0-9: a low half, b high half (empty AND); key 11 full in both
        low = (a & 0xFFFF) < 32768
        a = np.concatenate([a[(a >> 16 >= 10) | low], np.arange(11 << 16, 12 << 16)]).astype(np.uint32)
        b = np.nonzero(rng.random(U) < 0.4)[0].astype(np.uint32)
        b = np.concatenate([b[(b >> 16 >= 10) | ((b & 0xFFFF) >= 32768)], np.arange(11 << 16, 12 << 16)])
        a, b = np.unique(a), np.unique(b.astype(np.uint32))
    oa, ob = orc.upload_from_ids(a, U), orc.upload_from_ids(b, U)
    ga, gb = gpu.upload_from_ids(a, U), gpu.upload_from_ids(b, U)
    assert ga.n_containers == gb.n_containers == ga.max_key + 1 == 40
    want = orc.set_operation(oa, ob, op)
    g = gpu.set_operation(ga, gb, op)
    assert_same(gpu.download(g), want, strict=True, what=f"dense {case}")
    for x in (g, ga, gb):
        gpu.free(x)


def _irregular_run_operands():
    """Run containers as the portable format allows but run_optimize never
    writes: runs that touch (not merged), overlap, come out of order, or end past
    0xFFFF, and runs on word and chunk edges; each against an array, a bitmap,
    another run container, or nothing."""
    rng = np.random.default_rng(91)

    def run(*pairs):
        return (orc.TC_RUN, len(pairs), np.array(pairs, dtype=np.uint16).ravel())

    def arr(n):
        v = np.unique(rng.integers(0, 65536, n)).astype(np.uint16)
        return (orc.TC_ARRAY, v.size, v)

    def bmp(p):
        w = np.packbits(rng.random(65536) < p, bitorder="little").view(np.uint64)
        return (orc.TC_BITSET, int(np.unpackbits(w.view(np.uint8)).sum()) % 65536, w)

    many = [(2 * i * 7, i % 3) for i in range(3000)]  # 3000 short disjoint runs
    a = {0: run((100, 49), (150, 9), (160, 0)),            # touching
         1: run((1000, 500), (1200, 100), (1250, 3000)),   # overlapping
         2: run((5000, 10), (100, 20)),                     # out of order
         3: run((65000, 1000)),                             # ends past 0xFFFF
         4: run(*many),
         5: run((0, 0), (31, 1), (63, 64), (4095, 4097), (65535, 0)),
         6: run((7, 3)),                                    # one-sided
         8: run((31, 0), (32, 31), (64, 63), (127, 128)),   # touching on word edges
         9: run((9000, 10), (100, 20), (50, 70), (3000, 5), (2990, 20), (65000, 900)),  # > 4, unordered
         10: run(*[(i * 300, 299) for i in range(6)])}       # > 4, each touching the next
    b = {0: arr(300), 1: bmp(0.4), 2: run((90, 5), (96, 3)), 3: run((0, 65535)), 4: arr(4000),
         5: run((40000, 100), (30000, 5000)), 7: run((1, 1)), 8: bmp(0.02), 9: bmp(0.3),
         10: run((5, 1), (1000, 2), (4000, 3), (7000, 4), (9000, 5), (20000, 6))}
    to_list = lambda d: [(k,) + d[k] for k in sorted(d)]
    return to_list(a), to_list(b)


@pytest.mark.parametrize("op", [orc.AND, orc.OR, orc.ANDNOT, orc.XOR])
@pytest.mark.parametrize("swap", [False, True])
def test_set_operation_irregular_runs(gpu, op, swap):
    """Runs are decoded as the reference's expansion does (each run's bits
    ORed in, the end clamped to 0xFFFF; src/set_ops.cu:322-368) whatever their
    order: the decode by toggles, and its fallback for runs that are not sorted
    and disjoint."""
    _say("set_operation irregular runs", op, swap)
    ca, cb = _irregular_run_operands()
    if swap:
        ca, cb = cb, ca
    thr = orc.PROMOTE_KEEP_DEFAULT
    oa, ob = orc.upload_containers(ca, threshold=thr), orc.upload_containers(cb, threshold=thr)
    ga, gb = gpu.upload_containers(ca, 0, False, 0, thr), gpu.upload_containers(cb, 0, False, 0, thr)
    assert_same(gpu.download(ga), oa, strict=True, what="irregular upload a")
    assert_same(gpu.download(gb), ob, strict=True, what="irregular upload b")
    g = gpu.set_operation(ga, gb, op)
    assert_same(gpu.download(g), orc.set_operation(oa, ob, op), strict=True, what=f"irregular runs {op}")
    for x in (g, ga, gb):
        gpu.free(x)


def test_set_operation_empty_and_identical(gpu):
    _say("set_operation empty/identical")
    a = orc.Lite.from_sorted_ids(np.arange(1000, dtype=np.uint32))
    b = orc.Lite.from_sorted_ids(np.arange(65536, 66536, dtype=np.uint32))
    ga, _ = _upload_pair(gpu, a, 0, orc.PROMOTE_AUTO)
    gb, _ = _upload_pair(gpu, b, 0, orc.PROMOTE_AUTO)
    r = gpu.set_operation(ga, gb, orc.AND)
    assert r.n_containers == 0
    x = gpu.set_operation(ga, ga, orc.XOR)
    assert x.n_containers == 0 and x.n_bitmap_containers == 1  # array x array XOR -> mixed -> BITMAP slot
    e = gpu.upload_from_ids(np.zeros(0, np.uint32), 1000)
    r2 = gpu.set_operation(e, e, orc.OR)
    assert r2.n_containers == 0 and r2.universe_size == 1000
    for g in (r, x, r2, ga, gb, e):
        gpu.free(g)


# ---- multi_and ----------------------------------------------------------------
@pytest.mark.parametrize("case", ["fused_plain", "fused_negated", "fused_all_negated", "pairwise_arrays",
                                  "fused_absent_negated_key", "single", "fused_8", "fused_32", "pairwise_33"])
def test_multi_and_parity(gpu, case):
    _say("multi_and", case)
    rng = np.random.default_rng(sum(map(ord, case)))
    if case == "fused_absent_negated_key":  # test/test_complement.cu:604-679
        U = 3 * 65536
        la = np.nonzero(rng.random(U) < 0.2)[0]
        lb = np.setdiff1d(np.arange(U), [70000, 70001, 70005, 70100, 70200])
        lc = np.concatenate([np.nonzero(rng.random(65536) < 1 / 7)[0], 131072 + np.nonzero(rng.random(65536) < 1 / 7)[0]])
        logicals, thr = [la, lb, lc], orc.PROMOTE_ALL
    elif case == "fused_8":
        U = 8 * 65536
        logicals = [np.nonzero(rng.random(U) < (0.2 if i % 2 == 0 else 0.85))[0] for i in range(8)]
        thr = orc.PROMOTE_ALL
    elif case in ("fused_32", "pairwise_33"):  # the fused path's largest k (src/set_ops.cu:1715-1745), then one more
        k = 32 if case == "fused_32" else 33
        U = 4 * 65536
        # dense sets (most above U/2: complemented) so that the AND is not empty
        logicals = [np.nonzero(rng.random(U) < (0.97 if i % 4 else 0.6))[0] for i in range(k)]
        thr = orc.PROMOTE_ALL
    else:
        U = 200000
        dens = {"fused_plain": [0.6, 0.5, 0.4], "fused_negated": [0.33, 0.5, 0.75],
                "fused_all_negated": [0.75, 0.67, 0.8], "pairwise_arrays": [0.6, 0.01, 0.5],
                "single": [0.3]}[case]
        logicals = [np.nonzero(rng.random(U) < d)[0] for d in dens]
        thr = orc.PROMOTE_ALL if case in ("fused_negated", "fused_all_negated") else orc.PROMOTE_AUTO
    lites = [orc.Lite.from_sorted_ids(np.asarray(l, dtype=np.uint32)) for l in logicals]
    gs, os_ = [], []
    for lt in lites:
        want = orc.upload_packed(lt, U, thr, auto_l2(gpu))
        src, comp = (lt.flip(0, U), True) if lt.cardinality() > U // 2 else (lt, False)
        gs.append(gpu.upload_containers(src.containers(), U, comp, lt.cardinality(), thr))
        os_.append(want)
        assert_same(gpu.download(gs[-1]), want, strict=True, what="multi_and input")
    want = orc.multi_and(os_)
    g = gpu.multi_and(gs)
    assert_same(gpu.download(g), want, strict=True, what=f"multi_and {case}")
    for x in gs + [g]:
        gpu.free(x)


# ---- point queries ------------------------------------------------------------
QUERY_CASES = [("ids", 1 << 24, 0.01), ("ids", 1 << 24, 0.6), ("keep", 1 << 22, 0.001), ("keep", 1 << 22, 0.3),
               ("runs", 1 << 20, 0.0), ("bitset_neg", 1 << 21, 0.8), ("empty", 1 << 20, 0.0),
               ("small", 5000, 0.1), ("setop", 1 << 22, 0.002)]


@pytest.mark.parametrize("layout,universe,density", QUERY_CASES)
@pytest.mark.parametrize("mode", [0, 1, 2, 3, 4])
def test_contains_parity(gpu, layout, universe, density, mode):
    _say("contains", layout, universe, density, mode)
    torch = _torch()
    rng = np.random.default_rng(int(universe * 7 + density * 1000))
    ids = np.nonzero(rng.random(universe) < density)[0].astype(np.uint32)
    if layout == "ids":
        g, want = gpu.upload_from_ids(ids, universe), orc.upload_from_ids(ids, universe)
    elif layout == "keep":
        lt = orc.Lite.from_sorted_ids(ids)
        g = gpu.upload_containers(lt.containers(), universe, False, lt.cardinality(), orc.PROMOTE_KEEP_DEFAULT)
        want = orc.upload_packed(lt, universe, orc.PROMOTE_KEEP_DEFAULT)
    elif layout == "runs":
        ids = np.concatenate([np.arange(1000, 5000), np.arange(70000, 80000), np.arange(200000, 262144)]).astype(np.uint32)
        lt = orc.Lite.from_sorted_ids(ids).run_optimize()
        g = gpu.upload_containers(lt.containers(), 0, False, 0, orc.PROMOTE_KEEP_DEFAULT)
        want = orc.upload_packed(lt, None, orc.PROMOTE_KEEP_DEFAULT)
    elif layout == "bitset_neg":
        w = flat_from_ids(ids, universe)
        g, want = gpu.upload_from_bitset(w, universe), orc.upload_from_bitset(w, universe)
    elif layout == "setop":  # a set-operation result: no key_index, containers found by a search of keys
        half = np.nonzero(rng.random(universe) < 0.3)[0].astype(np.uint32)
        half = half[(half >> 16) % 3 == 0]  # bitmaps in every third key, arrays (ids) elsewhere
        la, lb = orc.Lite.from_sorted_ids(ids), orc.Lite.from_sorted_ids(half)
        ga = gpu.upload_containers(la.containers(), universe, False, la.cardinality(), orc.PROMOTE_KEEP_DEFAULT)
        gb = gpu.upload_containers(lb.containers(), universe, False, lb.cardinality(), orc.PROMOTE_KEEP_DEFAULT)
        oa = orc.upload_packed(la, universe, orc.PROMOTE_KEEP_DEFAULT)
        ob = orc.upload_packed(lb, universe, orc.PROMOTE_KEEP_DEFAULT)
        g, want = gpu.set_operation(ga, gb, orc.OR), orc.set_operation(oa, ob, orc.OR)
        gpu.free(ga)
        gpu.free(gb)
        assert not g.key_index and g.n_array_containers > 0 and g.n_bitmap_containers > 0
    elif layout == "empty":
        lt = orc.Lite.from_sorted_ids(np.zeros(0, np.uint32))
        g = gpu.upload_containers([], 0, False, 0, orc.PROMOTE_AUTO)
        want = orc.upload_packed(lt, None)
    else:
        g, want = gpu.upload_from_ids(ids, universe, orc.PROMOTE_KEEP_DEFAULT), orc.upload_from_ids(ids, universe, orc.PROMOTE_KEEP_DEFAULT)
    # uniform queries over 2x the universe, plus a clustered sorted block
    q = np.concatenate([rng.integers(0, 2 * max(universe, 1), 200000, dtype=np.uint64).astype(np.uint32),
                        np.sort(rng.integers(0, 65536, 8192, dtype=np.uint32)) + (universe // 2 & ~0xFFFF)])
    dq = _dev_u32(q)
    out = torch.empty_like(dq)
    gpu.contains_batch(g, dq, out, mode)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint32)
    assert np.array_equal(got, orc.contains_many(want, q))
    gpu.free(g)


# ---- randomized sweep over the tile-sort paths -------------------------------
def _sweep_case(i):
    """Case i of a seeded sweep: a universe, an id distribution (uniform,
    sorted, clustered windows, a few hot keys) and a size around the tile
    sort's 24576-id tiles and 8-tile blocks."""
    rng = np.random.default_rng(1000 + i)
    U = int(rng.choice([70000, 1 << 20, (1 << 22) + 5, 1 << 26, 1 << 30, 0xFFFFFFFF]))
    n = int(rng.choice([1025, 24575, 24577, 8 * 24576 + 3, 200_000, 700_000]))
    kind = ["uniform", "sorted", "windows", "hot"][i % 4]
    if kind == "uniform":
        ids = rng.integers(0, U, n, dtype=np.uint64)
    elif kind == "sorted":
        ids = np.sort(rng.integers(0, U, n, dtype=np.uint64))
    elif kind == "windows":  # runs of sorted ids in random 65536-aligned windows
        w = rng.integers(0, max(1, U >> 16), (n + 4095) // 4096, dtype=np.uint64)
        off = np.sort(rng.integers(0, 65536, ((n + 4095) // 4096, 4096), dtype=np.uint64), axis=1)
        ids = ((w[:, None] << 16) + off).reshape(-1)[:n] % U
    else:  # most ids in three keys, the rest uniform
        hot = rng.integers(0, max(1, U >> 16), 3, dtype=np.uint64)
        ids = np.where(rng.random(n) < 0.8, (hot[rng.integers(0, 3, n)] << 16) + rng.integers(0, 65536, n, dtype=np.uint64),
                       rng.integers(0, U, n, dtype=np.uint64)) % U
    return U, kind, ids.astype(np.uint32), rng


@pytest.mark.parametrize("i", range(16))
def test_tile_sort_paths_random_sweep(gpu, i):
    """upload_from_device_ids (strict, against the oracle) and partitioned
    queries (the ids themselves, the ids + 1, and uniform queries past U)."""
    U, kind, ids, rng = _sweep_case(i)
    _say("tile-sort sweep", i, U, kind, ids.size)
    torch = _torch()
    want = orc.upload_from_ids(ids, U, orc.PROMOTE_AUTO, auto_l2(gpu))
    g = gpu.upload_from_device_ids(_dev_u32(ids), U)
    assert_same(gpu.download(g), want, strict=True, what=f"sweep {i} {kind}")
    q = np.concatenate([ids, ids + np.uint32(1), rng.integers(0, 0xFFFFFFFF, 30_001, dtype=np.uint64).astype(np.uint32)])
    out = torch.empty(q.size, dtype=torch.int32, device="cuda")
    gpu.contains_batch(g, _dev_u32(q), out, 4)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), orc.contains_many(want, q)), (i, kind)
    gpu.free(g)

"""Pins the oracle's restatement of the reference (CPU only).

Each test follows a known-answer test of the reference suite (cited) or checks
the restatement against an independent flat-bitset brute force.  The flat
bitset is built from the input ids with numpy, never from oracle code.
"""
import numpy as np
import pytest

import orc
from helpers import assert_same, flat_from_ids, ids_from_flat, mt_bernoulli, mt_mod_filter, mt_low16_density, words_mask

L2 = orc.DEFAULT_L2


# ---- resolve_auto_threshold (test/test_promote.cu:257-381) ----------------
def test_auto_threshold_pinned_verdicts():
    assert orc.resolve_auto_threshold(1_000_000) == orc.PROMOTE_KEEP_DEFAULT
    assert orc.resolve_auto_threshold(1_000_000_000) == orc.PROMOTE_ALL
    assert orc.resolve_auto_threshold(100_000) == orc.PROMOTE_KEEP_DEFAULT
    assert orc.resolve_auto_threshold(1 << 30) == orc.PROMOTE_ALL
    assert orc.resolve_auto_threshold(10_000) == orc.PROMOTE_KEEP_DEFAULT
    assert orc.resolve_auto_threshold(0) == orc.PROMOTE_KEEP_DEFAULT


def test_auto_threshold_crossover_is_flat_times_two_over_l2():
    # flat = ceil(U/8); promote iff 2*flat > L2 (strict).  With 4 MiB: U = 2^24 keeps.
    assert orc.resolve_auto_threshold(1 << 24, L2) == orc.PROMOTE_KEEP_DEFAULT
    assert orc.resolve_auto_threshold((1 << 24) + 1, L2) == orc.PROMOTE_ALL
    assert orc.resolve_auto_threshold((1 << 24) + 8, L2) == orc.PROMOTE_ALL
    # a 256 MiB cache would keep 2^30 (the verdict the reference test forbids)
    assert orc.resolve_auto_threshold(1 << 30, 256 << 20) == orc.PROMOTE_KEEP_DEFAULT


# ---- upload_from_ids known answers -----------------------------------------
def test_upload_unsorted_duplicates():  # test/test_promote.cu:387-416
    ids = [200, 5, 100000, 42, 65536, 0, 100000, 5]
    r = orc.upload_from_ids(ids, 200000, orc.PROMOTE_KEEP_DEFAULT)
    assert r.total_cardinality == 6
    bs = orc.decompress(r)
    bit = lambda i: (int(bs[i // 32]) >> (i % 32)) & 1
    for i in (0, 5, 42, 200, 65536, 100000):
        assert bit(i) == 1
    for i in (1, 100, 65535):
        assert bit(i) == 0


def test_upload_all_duplicates():  # :418-429
    r = orc.upload_from_ids([42] * 4, 100, orc.PROMOTE_KEEP_DEFAULT)
    assert r.total_cardinality == 1 and r.n_containers == 1


def test_upload_reversed():  # :431-449  (1000 of 1000 -> negated, empty stored set)
    r = orc.upload_from_ids(np.arange(999, -1, -1), 1000, orc.PROMOTE_KEEP_DEFAULT)
    assert r.total_cardinality == 1000
    assert r.negated and r.n_containers == 0
    assert int(np.unpackbits(orc.decompress(r).view(np.uint8)).sum()) == 1000


def test_upload_threshold_keep_and_all():  # :183-218
    ids = np.array([k * 65536 + j * 100 for k in range(5) for j in range(100)], dtype=np.uint32)
    arr = orc.upload_from_ids(ids, 5 * 65536, orc.PROMOTE_KEEP_DEFAULT)
    assert (arr.n_containers, arr.n_array_containers, arr.n_bitmap_containers) == (5, 5, 0)
    bmp = orc.upload_from_ids(ids, 5 * 65536, orc.PROMOTE_ALL)
    assert (bmp.n_containers, bmp.n_bitmap_containers, bmp.n_array_containers) == (5, 5, 0)
    assert np.array_equal(orc.decompress(arr), orc.decompress(bmp))
    assert np.array_equal(orc.decompress(arr), flat_from_ids(ids, 5 * 65536))


def test_upload_custom_threshold():  # :220-251
    ids = np.array([k * 65536 + j for k in range(3) for j in range(200)], dtype=np.uint32)
    bmp = orc.upload_from_ids(ids, 3 * 65536, 100)
    assert (bmp.n_bitmap_containers, bmp.n_array_containers) == (3, 0)
    arr = orc.upload_from_ids(ids, 3 * 65536, orc.PROMOTE_KEEP_DEFAULT)
    assert (arr.n_array_containers, arr.n_bitmap_containers) == (3, 0)
    assert np.array_equal(orc.decompress(arr), orc.decompress(bmp))


def test_upload_auto_small_and_large():  # :269-381
    ids = np.arange(500, dtype=np.uint32) * 100
    bm = orc.upload_from_ids(ids, 100000)
    assert bm.n_array_containers > 0
    small = orc.upload_from_ids([0, 100, 200], 10000)
    assert (small.n_array_containers, small.n_bitmap_containers) == (1, 0)
    large = orc.upload_from_ids([0, 100, 200], 1_000_000_000)
    assert (large.n_bitmap_containers, large.n_array_containers) == (1, 0)
    three = orc.upload_from_ids([0, 65536, 131072], 1_000_000_000)
    assert (three.n_bitmap_containers, three.n_array_containers) == (3, 0)


def _check_contains(r, universe, ids, step):
    truth = np.zeros(universe, dtype=bool)
    truth[np.asarray(ids, dtype=np.int64)] = True
    q = np.arange(0, universe, step, dtype=np.uint32)
    got = orc.contains_many(r, q).astype(bool)
    assert np.array_equal(got, truth[q])


def test_negated_contains_small():  # test/test_complement.cu:129-149
    ids = [0, 1, 2, 3, 4, 5, 6, 8, 9]
    r = orc.upload_from_ids(ids, 10)
    assert r.negated
    _check_contains(r, 10, ids, 1)
    assert r.n_containers == 1 and r.cards[0] == 1  # stores {7}


def test_negated_contains_absent_key():  # :151-182
    ids = mt_mod_filter(42, 200000, 10, keep_zero=False)
    r = orc.upload_from_ids(ids, 200000)
    assert r.negated
    _check_contains(r, 200000, ids, 7)


def test_negated_contains_large_gpu_path():  # :184-210
    ids = mt_mod_filter(123, 100000, 5, keep_zero=False)
    assert ids.size > 1024
    r = orc.upload_from_ids(ids, 100000)
    assert r.negated
    _check_contains(r, 100000, ids, 3)


def test_no_negate_low_density_and_exact_half():  # :212-237
    ids = mt_mod_filter(42, 100000, 10, keep_zero=True)
    assert not orc.upload_from_ids(ids, 100000).negated
    assert not orc.upload_from_ids(np.arange(50), 100).negated


def test_decompress_negated():  # :282-313
    ids = np.array([i for i in range(50000) if i % 5 != 0], dtype=np.uint32)
    r = orc.upload_from_ids(ids, 50000)
    assert r.negated
    assert np.array_equal(orc.decompress(r), flat_from_ids(ids, 50000))


@pytest.mark.parametrize("n,universe,seed", [(600, 1 << 20, 1), (1024, 70000, 2), (1025, 70000, 3),
                                             (5000, 1 << 22, 4), (20000, 300000, 5), (60000, 100000, 6)])
def test_upload_ids_layout_bruteforce(n, universe, seed):
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, universe, n, dtype=np.uint32)
    r = orc.upload_from_ids(ids, universe, orc.PROMOTE_KEEP_DEFAULT)
    uniq = np.unique(ids)
    assert r.total_cardinality == uniq.size
    assert np.array_equal(orc.decompress(r), flat_from_ids(uniq, universe))
    assert np.all(np.diff(r.keys.astype(np.int64)) > 0)
    if n > 1024:  # GPU path: all bitmap, dense offsets, key_index from U
        assert r.n_bitmap_containers == r.n_containers and r.n_array_containers == 0
        assert np.array_equal(r.offsets, np.arange(r.n_containers, dtype=np.uint32) * 8192)
        assert r.max_key == (universe - 1) >> 16
        assert r.key_index.size == r.max_key + 1
    stored = uniq if not r.negated else np.setdiff1d(np.arange(universe, dtype=np.uint32), uniq)
    counts = np.bincount(stored >> 16, minlength=65536)
    for i, k in enumerate(r.keys):
        c = counts[k]
        assert r.cards[i] == (0 if c > 65535 else c)
        assert r.key_index[k] == i


def test_upload_ids_full_container_card_wraps():  # Q2: 65536 stored as 0 (upload_ids.cu:105)
    ids = np.arange(65536 * 2 + 100, dtype=np.uint32)
    r = orc.upload_from_ids(ids, 1 << 22)
    assert list(r.cards) == [0, 0, 100]
    assert orc.true_cardinality(r) == ids.size


# ---- bitset uploads (test/test_complement.cu:793-908) ---------------------
def _bitset(ids, universe):
    return flat_from_ids(ids, universe)


def test_bitset_sparse_dense_roundtrip():
    U = 100000
    sparse = mt_mod_filter(42, U, 10, keep_zero=True)
    r = orc.upload_from_bitset(_bitset(sparse, U), U)
    assert not r.negated
    _check_contains(r, U, sparse, 7)
    dense = mt_mod_filter(42, U, 10, keep_zero=False)
    r = orc.upload_from_bitset(_bitset(dense, U), U)
    assert r.negated and r.total_cardinality == dense.size
    _check_contains(r, U, dense, 3)
    U2 = 200000
    third = mt_mod_filter(99, U2, 3, keep_zero=True)
    bs = _bitset(third, U2)
    r = orc.upload_from_bitset(bs, U2)
    assert np.array_equal(words_mask(orc.decompress(r, bs.size), U2), words_mask(bs, U2))
    quarter = mt_mod_filter(42, U, 4, keep_zero=True)
    r = orc.upload_from_bitset(_bitset(quarter, U), U)
    assert not r.negated
    _check_contains(r, U, quarter, 11)


def test_bitset_layout_rules():
    U = 5 * 65536 + 123
    rng = np.random.default_rng(7)
    ids = np.concatenate([rng.integers(0, 65536, 50), 3 * 65536 + rng.integers(0, 65536, 10)]).astype(np.uint32)
    bs = _bitset(ids, U)
    r = orc.upload_from_bitset(bs, U)
    assert list(r.keys) == [0, 3]  # empty chunks skipped, always BITMAP
    assert list(r.types) == [orc.BITMAP, orc.BITMAP]
    assert r.max_key == 3 and r.key_index.size == 4  # last non-empty chunk
    # a 90% bitset negates: stored complement, tail word masked
    dense = np.setdiff1d(np.arange(U, dtype=np.uint32), ids)
    r = orc.upload_from_bitset(_bitset(dense, U), U)
    assert r.negated and r.total_cardinality == dense.size
    assert np.array_equal(words_mask(orc.decompress(r), U), words_mask(_bitset(dense, U), U))


def test_bitset_empty_words():
    r = orc.upload_from_bitset(np.zeros(0, dtype=np.uint32), 1000)
    assert r.n_containers == 0 and r.universe_size == 1000


# ---- set operations ---------------------------------------------------------
def _truth_op(a, b, op):
    return {orc.AND: a & b, orc.OR: a | b, orc.ANDNOT: a & ~b, orc.XOR: a ^ b}[op]


def _make_demorgan(density, seed, force_negate, U=100000):
    """DeMorganTest::make_bitmap (test/test_complement.cu:372-398)."""
    logical = mt_bernoulli(seed, density, U)
    lite = orc.Lite.from_sorted_ids(logical)
    if force_negate:
        comp = lite.flip(0, U)
        r = orc.upload_packed(comp)  # upload() without universe
        r.negated = True
        r.universe_size = U
        r.total_cardinality = logical.size
        r._c = None
    else:
        r = orc.upload_packed(lite, U)
    return r, logical


@pytest.mark.parametrize("op", [orc.AND, orc.OR, orc.ANDNOT, orc.XOR])
@pytest.mark.parametrize("na", [False, True])
@pytest.mark.parametrize("nb", [False, True])
def test_demorgan_16(op, na, nb):  # test/test_complement.cu:400-462
    U = 100000
    a, la = _make_demorgan(0.3, 42, na)
    b, lb = _make_demorgan(0.4, 99, nb)
    r = orc.set_operation(a, b, op)
    want = words_mask(_truth_op(flat_from_ids(la, U), flat_from_ids(lb, U), op), U)
    assert np.array_equal(words_mask(orc.decompress(r, (U + 31) // 32), U), want)
    assert r.total_cardinality == 0 and r.key_index is None and r.max_key == 0  # Q3


def test_setop_user_example():  # :320-359
    a = orc.upload_from_ids([0, 1, 2, 3, 4, 5, 6, 8, 9], 10)
    b = orc.upload_from_ids([4, 6, 7], 10)
    assert a.negated and not b.negated
    r = orc.set_operation(a, b, orc.AND)
    assert list(ids_from_flat(words_mask(orc.decompress(r, 1), 10))) == [4, 6]


def _lite_random(U, density, seed):
    return orc.Lite.from_sorted_ids(mt_bernoulli(seed, density, U))


@pytest.mark.parametrize("case", [("AND", 0.6, 100, 0.4, 200), ("AND", 0.02, 300, 0.01, 400),
                                  ("AND", 0.5, 500, 0.02, 600), ("OR", 0.5, 800, 0.3, 900),
                                  ("ANDNOT", 0.5, 1000, 0.3, 1100), ("XOR", 0.5, 1200, 0.3, 1300)])
def test_set_ops_suite(case):  # test/test_set_ops.cu:84-266
    name, da, sa, db, sb = case
    op = getattr(orc, name)
    U = 200000
    la, lb = mt_bernoulli(sa, da, U), mt_bernoulli(sb, db, U)
    a = orc.upload_packed(orc.Lite.from_sorted_ids(la))
    b = orc.upload_packed(orc.Lite.from_sorted_ids(lb))
    r = orc.set_operation(a, b, op)
    n_words = (r.universe_size + 31) // 32
    want = _truth_op(flat_from_ids(la, U, n_words), flat_from_ids(lb, U, n_words), op)
    assert np.array_equal(orc.decompress(r, n_words), want)


def test_set_ops_empty_and_identical():  # :144-162, :269-285
    a = orc.upload_packed(orc.Lite.from_sorted_ids(np.arange(1000, dtype=np.uint32)))
    b = orc.upload_packed(orc.Lite.from_sorted_ids(np.arange(65536, 66536, dtype=np.uint32)))
    assert orc.set_operation(a, b, orc.AND).n_containers == 0
    x = mt_bernoulli(1400, 0.4, 100000)
    xa = orc.upload_packed(orc.Lite.from_sorted_ids(x))
    xb = orc.upload_packed(orc.Lite.from_sorted_ids(x))
    assert orc.set_operation(xa, xb, orc.XOR).n_containers == 0
    same = orc.set_operation(xa, xb, orc.AND)
    assert np.array_equal(orc.decompress(same), flat_from_ids(x, same.universe_size))


def test_set_ops_output_types_and_slots():  # Q4/Q5 layout rules
    U = 4 * 65536
    dense = np.arange(0, 65536, 2, dtype=np.uint32)  # bitmap in key 0
    sparse = np.array([2, 4, 6, 65536 + 3, 2 * 65536 + 1], dtype=np.uint32)  # arrays in keys 0,1,2
    run = orc.Lite.from_sorted_ids(np.arange(3 * 65536, 3 * 65536 + 5000, dtype=np.uint32)).run_optimize()
    A = orc.upload_packed(orc.Lite.from_sorted_ids(dense).op(run, orc.OR).run_optimize(), U, orc.PROMOTE_KEEP_DEFAULT)
    B = orc.upload_packed(orc.Lite.from_sorted_ids(sparse), U, orc.PROMOTE_KEEP_DEFAULT)
    assert A.n_run_containers == 1 and B.n_array_containers == 3
    r_and = orc.set_operation(A, B, orc.AND)
    assert list(r_and.keys) == [0] and list(r_and.types) == [orc.ARRAY]  # ba -> ARRAY, run-less keys dropped
    r_or = orc.set_operation(A, B, orc.OR)
    assert list(r_or.keys) == [0, 1, 2, 3]
    assert list(r_or.types) == [orc.BITMAP, orc.ARRAY, orc.ARRAY, orc.RUN]  # mixed->BITMAP, copies keep type
    assert r_or.n_bitmap_containers == 1 and r_or.n_array_containers == 2 and r_or.n_run_containers == 1
    r_x = orc.set_operation(A, A, orc.XOR)  # bb and run x run both empty -> dropped, slots still counted
    assert r_x.n_containers == 0 and r_x.n_bitmap_containers == 2
    truth = flat_from_ids(np.union1d(np.union1d(dense, sparse), np.arange(3 * 65536, 3 * 65536 + 5000)), U)
    assert np.array_equal(orc.decompress(r_or), truth)


def test_set_ops_full_container_and_is_dropped():  # Q2 x Q4: 65536 -> card 0 -> dropped
    full = orc.upload_from_ids(np.arange(65536, dtype=np.uint32), 1 << 20)
    r = orc.set_operation(full, full, orc.AND)
    assert r.n_containers == 0 and r.n_bitmap_containers == 1
    r = orc.set_operation(full, full, orc.OR)
    assert r.n_containers == 1 and r.cards[0] == 0


# ---- multi_and (test/test_complement.cu:502-790) --------------------------
def _flat_and(logicals, U):
    acc = flat_from_ids(logicals[0], U)
    for l in logicals[1:]:
        acc &= flat_from_ids(l, U)
    return acc


def test_multi_and_with_negated():
    U = 50000
    g = orc.mt_raw(42, 3 * U).reshape(U, 3)
    l1 = np.nonzero(g[:, 0] % 3 == 0)[0].astype(np.uint32)
    l2 = np.nonzero(g[:, 1] % 2 == 0)[0].astype(np.uint32)
    l3 = np.nonzero(g[:, 2] % 4 != 0)[0].astype(np.uint32)
    ins = [orc.upload_packed(orc.Lite.from_sorted_ids(l), U) for l in (l1, l2, l3)]
    assert ins[2].negated
    r = orc.multi_and(ins)
    assert r.n_array_containers == 0 and r.key_index is not None  # fused path
    assert np.array_equal(words_mask(orc.decompress(r, (U + 31) // 32), U), words_mask(_flat_and([l1, l2, l3], U), U))


def test_multi_and_all_negated():
    U = 200000
    g = orc.mt_raw(77, 3 * U).reshape(U, 3)
    ls = [np.nonzero(g[:, 0] % 4 != 0)[0], np.nonzero(g[:, 1] % 3 != 0)[0], np.nonzero(g[:, 2] % 5 != 0)[0]]
    ins = [orc.upload_packed(orc.Lite.from_sorted_ids(l.astype(np.uint32)), U) for l in ls]
    assert all(r.negated for r in ins)
    r = orc.multi_and(ins)
    # The tail key (196608..199999) stores ~850 complement ids -> an ARRAY container, so
    # multi_and routes pairwise (src/set_ops.cu:1726-1735) despite the test's comment.
    assert any(x.n_array_containers for x in ins) and r.key_index is None and r.negated
    assert np.array_equal(words_mask(orc.decompress(r, (U + 31) // 32), U), words_mask(_flat_and(ls, U), U))
    # Forced all-bitmap inputs take the fused path: keys [0, ceil(U/65536)) = 0..3.
    ins = [orc.upload_packed(orc.Lite.from_sorted_ids(l.astype(np.uint32)), U, orc.PROMOTE_ALL) for l in ls]
    r = orc.multi_and(ins)
    assert list(r.keys) == [0, 1, 2, 3] and r.max_key == 3 and not r.negated
    assert np.array_equal(words_mask(orc.decompress(r, (U + 31) // 32), U), words_mask(_flat_and(ls, U), U))


def test_fused_absent_key_in_negated_input():
    U = 3 * 65536
    g = orc.mt_raw(1001, 3 * 65536 + 2 * 65536)
    la = np.nonzero(g[:U] % 5 == 0)[0].astype(np.uint32)
    rest = g[U:].reshape(65536, 2)
    lc = np.concatenate([np.nonzero(rest[:, 0] % 7 == 0)[0], 131072 + np.nonzero(rest[:, 1] % 7 == 0)[0]])
    lc = np.sort(lc).astype(np.uint32)
    lb = np.setdiff1d(np.arange(U, dtype=np.uint32), np.array([70000, 70001, 70005, 70100, 70200], dtype=np.uint32))
    A = orc.upload_packed(orc.Lite.from_sorted_ids(la), U, orc.PROMOTE_ALL)
    B = orc.upload_packed(orc.Lite.from_sorted_ids(lb), U, orc.PROMOTE_ALL)
    C = orc.upload_packed(orc.Lite.from_sorted_ids(lc), U, orc.PROMOTE_ALL)
    assert B.negated and B.n_containers == 1  # :643-644
    assert not A.negated and not C.negated and A.n_array_containers == 0 and C.n_array_containers == 0
    r = orc.multi_and([A, B, C])
    want = words_mask(_flat_and([la, lb, lc], U), U)
    assert np.array_equal(words_mask(orc.decompress(r, (U + 31) // 32), U), want)
    assert want.any()


def test_fused_mixed_negation_many_containers():
    U = 16 * 65536
    g = orc.mt_raw(2002, 5 * U).reshape(5, U)
    dens = [0.30, 0.90, 0.15, 0.75, 0.25]
    ls = [np.nonzero(mt_low16_density(g[i], d))[0].astype(np.uint32) for i, d in enumerate(dens)]
    ins = [orc.upload_packed(orc.Lite.from_sorted_ids(l), U, orc.PROMOTE_ALL) for l in ls]
    assert [r.negated for r in ins] == [False, True, False, True, False]
    r = orc.multi_and(ins)
    want = words_mask(_flat_and(ls, U), U)
    assert np.array_equal(words_mask(orc.decompress(r, (U + 31) // 32), U), want)
    assert want.any()


def test_fused_alternating_8():
    U = 8 * 65536
    g = orc.mt_raw(3003, 8 * U).reshape(8, U)
    ls = [np.nonzero(mt_low16_density(g[i], 0.20 if i % 2 == 0 else 0.85))[0].astype(np.uint32) for i in range(8)]
    ins = [orc.upload_packed(orc.Lite.from_sorted_ids(l), U, orc.PROMOTE_ALL) for l in ls]
    assert [r.negated for r in ins] == [i % 2 == 1 for i in range(8)]
    r = orc.multi_and(ins)
    assert np.array_equal(words_mask(orc.decompress(r, (U + 31) // 32), U), words_mask(_flat_and(ls, U), U))


def test_multi_and_routing_and_card_clamp():
    full = np.arange(65536, dtype=np.uint32)
    a = orc.upload_from_ids(full, 1 << 20)
    b = orc.upload_from_ids(full, 1 << 20)
    r = orc.multi_and([a, b])
    assert r.n_containers == 1 and r.cards[0] == 65535 and r.total_cardinality == 65536  # clamp, Q7
    one = orc.multi_and([a])  # count == 1 -> set_operation(a, a, AND): full container dropped
    assert one.n_containers == 0
    assert orc.multi_and([]).n_containers == 0
    sparse = orc.upload_from_ids([1, 2, 3], 1 << 20, orc.PROMOTE_KEEP_DEFAULT)  # array -> pairwise chain
    r = orc.multi_and([a, b, sparse])
    # AND(a, b) drops the full container (card 65536 stored as 0), so the chain is empty
    assert r.key_index is None and r.n_containers == 0
    half = orc.upload_from_ids(np.arange(0, 65536, 2, dtype=np.uint32), 1 << 20)
    r = orc.multi_and([half, a, sparse])
    assert r.key_index is None and list(r.types) == [orc.ARRAY] and list(r.array_data[:1]) == [2]


# ---- next rows: enumerate_ids, promote_to_bitmap, deep copy ------------------
@pytest.mark.parametrize("kind", ["ids", "packed_mixed", "negated", "full_container"])
def test_enumerate_ids_is_the_sorted_stored_set(kind):
    """The expected list is built with numpy from the inputs: the unique ids, or
    for a negated result the complement that is stored."""
    rng = np.random.default_rng(5)
    if kind == "ids":
        ids = rng.integers(0, 1 << 22, 200000, dtype=np.uint64).astype(np.uint32)
        r, want = orc.upload_from_ids(ids, 1 << 22), np.unique(ids)
    elif kind == "packed_mixed":
        ids = np.unique(np.concatenate([rng.integers(0, 65536, 300, dtype=np.uint64),
                                        np.arange(65536, 65536 + 50000), np.arange(131072, 141072)]).astype(np.uint32))
        r, want = orc.upload_packed(orc.Lite.from_sorted_ids(ids).run_optimize(), None, orc.PROMOTE_KEEP_DEFAULT), ids
        assert r.n_run_containers > 0 and r.n_array_containers > 0
    elif kind == "negated":
        ids = np.arange(0, 90000, dtype=np.uint32)
        r, want = orc.upload_from_ids(ids, 100000), np.arange(90000, 100000)
        assert r.negated
    else:
        ids = np.arange(0, 3 * 65536 + 7, dtype=np.uint32)
        r, want = orc.upload_from_ids(ids, 1 << 20), ids
    got = orc.enumerate_ids(r)
    assert np.array_equal(got, want.astype(np.int64))


def test_enumerate_ids_set_operation_result_is_empty():  # total_cardinality left 0 (to_csr.cu:163)
    a = orc.upload_from_ids(np.arange(0, 5000, dtype=np.uint32), 1 << 20)
    b = orc.upload_from_ids(np.arange(2500, 7000, dtype=np.uint32), 1 << 20)
    r = orc.set_operation(a, b, orc.AND)
    assert r.total_cardinality == 0 and r.n_containers == 1
    assert orc.enumerate_ids(r).size == 0


def test_promote_mixed_containers():  # test/test_promote.cu:41-80
    ids = np.unique(np.concatenate([np.arange(100) * 10, np.arange(65536, 65536 + 50000),
                                    np.arange(131072, 141072)]).astype(np.uint32))
    g = orc.upload_packed(orc.Lite.from_sorted_ids(ids).run_optimize(), None, orc.PROMOTE_KEEP_DEFAULT)
    assert g.n_containers == 3 and g.n_array_containers + g.n_run_containers > 0
    p = orc.promote_to_bitmap(g)
    assert (p.n_containers, p.n_bitmap_containers, p.n_array_containers, p.n_run_containers) == (3, 3, 0, 0)
    assert np.array_equal(orc.decompress(p), orc.decompress(g))
    assert np.array_equal(p.offsets, np.arange(3, dtype=np.uint32) * 8192)
    assert np.array_equal(p.cards, g.cards)  # a RUN container keeps its n_runs
    assert p.max_key == (g.universe_size - 1) >> 16
    assert [int(p.key_index[k]) for k in range(3)] == [0, 1, 2]


def test_promote_all_bitmap_empty_and_arrays():  # :82-150
    g = orc.upload_packed(orc.Lite.from_sorted_ids(np.arange(3 * 65536, dtype=np.uint32)), None,
                          orc.PROMOTE_KEEP_DEFAULT)
    p = orc.promote_to_bitmap(g)
    assert p.n_bitmap_containers == 3 and np.array_equal(orc.decompress(p), orc.decompress(g))
    e = orc.promote_to_bitmap(orc.upload_packed(orc.Lite.from_sorted_ids(np.zeros(0, np.uint32)), None))
    assert e.n_containers == 0 and e.universe_size == 0  # GpuRoaring{} (promote.cu:236)
    rng = np.random.default_rng(42)
    ids = np.unique(np.concatenate([k * 65536 + rng.integers(0, 65536, 100) for k in range(50)]).astype(np.uint32))
    a = orc.upload_packed(orc.Lite.from_sorted_ids(ids), None, orc.PROMOTE_KEEP_DEFAULT)
    assert a.n_bitmap_containers == 0
    p = orc.promote_to_bitmap(a)
    assert p.n_bitmap_containers == p.n_containers == 50 and np.array_equal(orc.decompress(p), orc.decompress(a))


def test_promote_preserves_negated():  # test/test_complement.cu:468-497
    U = 100000
    ids = np.array([i for i in range(U) if i % 5], dtype=np.uint32)
    g = orc.upload_from_ids(ids, U)
    assert g.negated
    p = orc.promote_to_bitmap(g)
    assert p.negated and p.n_array_containers == 0
    q = np.arange(0, U, 13, dtype=np.uint32)
    assert np.array_equal(orc.contains_many(p, q), (q % 5 != 0).astype(np.uint32))


def test_deep_copy_and_promote_auto():
    rng = np.random.default_rng(9)
    ids = np.unique(rng.integers(0, 1 << 22, 3000, dtype=np.uint64).astype(np.uint32))
    g = orc.upload_packed(orc.Lite.from_sorted_ids(ids), 1 << 22, orc.PROMOTE_KEEP_DEFAULT)
    d = orc.deep_copy(g)
    assert_same(d, g, strict=False, what="deep_copy")
    assert d.bitmap_data.size == g.n_bitmap_containers * 1024
    # AUTO at 2^22 (512 KiB flat) keeps the layout on a 4 MiB L2; at 2^30 it promotes
    assert orc.promote_auto(g).n_array_containers == g.n_array_containers
    big = orc.upload_packed(orc.Lite.from_sorted_ids(ids), 1 << 30, orc.PROMOTE_KEEP_DEFAULT)
    p = orc.promote_auto(big)
    assert p.n_array_containers == 0 and p.n_bitmap_containers == p.n_containers


@pytest.mark.parametrize("seed", range(6))
def test_packed_upload_offsets_are_prefix_sums(seed):
    """The oracle's packed layout (src/upload.cpp:89-287) against what the layout
    itself fixes: each type's pool holds its containers in key order, back to
    back (helpers.assert_packed_offsets), for random mixes of array, bitmap and
    run containers, thresholds and complements; and the decoded set is the input's."""
    from helpers import assert_packed_offsets
    rng = np.random.default_rng(500 + seed)
    parts = []
    for key in range(int(rng.integers(1, 40))):
        base = int(rng.integers(0, 4096)) * 65536
        kind = int(rng.integers(0, 3))
        if kind == 0:
            parts.append(base + np.unique(rng.integers(0, 65536, int(rng.integers(1, 4000)))))
        elif kind == 1:
            parts.append(base + np.nonzero(rng.random(65536) < rng.uniform(0.1, 0.9))[0])
        else:
            s = int(rng.integers(0, 60000))
            parts.append(base + np.arange(s, s + int(rng.integers(1, 5000))))
    ids = np.unique(np.concatenate(parts)).astype(np.uint32)
    lite = orc.Lite.from_sorted_ids(ids).run_optimize()
    for thr in (orc.PROMOTE_KEEP_DEFAULT, orc.PROMOTE_ALL, 100):
        h = orc.upload_packed(lite, None, thr)
        assert_packed_offsets(h, what=f"seed {seed} thr {thr}")
        assert np.array_equal(orc.enumerate_ids(h), ids.astype(np.int64))
    U = int(ids.max()) + 1
    h = orc.upload_packed(lite, U, orc.PROMOTE_KEEP_DEFAULT)  # the complement when more than U/2
    assert_packed_offsets(h, what=f"seed {seed} with U")
    stored = orc.enumerate_ids(h)
    if h.negated:
        stored = np.setdiff1d(np.arange(U, dtype=np.int64), stored)
    assert np.array_equal(stored, ids.astype(np.int64))
    # a dense set: stored as its complement, whose pools obey the same rule
    U2 = 3 * 65536 + 777 + seed
    dense = np.setdiff1d(np.arange(U2), rng.integers(0, U2, 20000)).astype(np.uint32)
    h = orc.upload_packed(orc.Lite.from_sorted_ids(dense).run_optimize(), U2, orc.PROMOTE_KEEP_DEFAULT)
    assert h.negated
    assert_packed_offsets(h, what=f"seed {seed} complement")
    stored = np.setdiff1d(np.arange(U2, dtype=np.int64), orc.enumerate_ids(h))
    assert np.array_equal(stored, dense.astype(np.int64))

"""GPU parity of the fused filtered top-k against the closed-form oracle.

The oracle (orc.topk_bruteforce) computes exact fp64 squared L2 distances over
the passing ids and keeps the k smallest, ties broken by the smaller id.  The
GPU computes fp32 distances on MFMA tiles.  The bar: every returned distance
within 1e-4 relative of the fp64 distance of the returned id; distances
ascending; and the returned id set equal to the oracle's except for ids whose
distance ties the k-th distance within that tolerance.
"""
import numpy as np
import pytest

import orc
from helpers import mt_bernoulli

pytestmark = pytest.mark.gpu

RTOL = 1e-4


def _say(*a):
    print("CASE", *a, flush=True)


def _torch():
    import torch
    return torch


def _data(n_base, n_q, dim, seed):
    rng = np.random.default_rng(seed)
    base = rng.standard_normal((n_base, dim)).astype(np.float32)
    queries = rng.standard_normal((n_q, dim)).astype(np.float32)
    return base, queries


def _run(gpu, base, queries, k, filt):
    torch = _torch()
    db = torch.from_numpy(base).cuda()
    dq = torch.from_numpy(queries).cuda()
    dist = torch.empty((queries.shape[0], k), dtype=torch.float32, device="cuda")
    ids = torch.empty((queries.shape[0], k), dtype=torch.int64, device="cuda")
    gpu.topk_filtered(db, dq, k, filt, dist, ids)
    torch.cuda.synchronize()
    return dist.cpu().numpy(), ids.cpu().numpy()


def check_topk(base, queries, k, passing, got_d, got_i):
    want_d, want_i = orc.topk_bruteforce(base, queries, k, passing)
    n_pass = base.shape[0] if passing is None else int(np.count_nonzero(passing))
    valid = min(k, n_pass)
    for q in range(queries.shape[0]):
        gi, gd = got_i[q], got_d[q]
        assert np.all(gi[valid:] == -1) and np.all(np.isinf(gd[valid:])), f"query {q}: padding"
        gi, gd = gi[:valid], gd[:valid]
        assert np.all(gi >= 0) and np.all(gi < base.shape[0]), f"query {q}: id range"
        assert len(set(gi.tolist())) == valid, f"query {q}: duplicate ids"
        if passing is not None:
            assert np.all(passing[gi] != 0), f"query {q}: id outside the filter"
        exact = ((base[gi].astype(np.float64) - queries[q].astype(np.float64)) ** 2).sum(axis=1)
        assert np.allclose(gd, exact, rtol=RTOL, atol=0), f"query {q}: distance off by more than 1e-4 rel"
        assert np.all(np.diff(gd) >= 0), f"query {q}: not ascending"
        wi, wd = want_i[q][:valid], want_d[q][:valid]
        if valid == 0:
            continue
        kth = wd[-1]
        only_gpu = set(gi.tolist()) - set(wi.tolist())
        only_cpu = set(wi.tolist()) - set(gi.tolist())
        for i in only_gpu | only_cpu:
            di = float(((base[i].astype(np.float64) - queries[q].astype(np.float64)) ** 2).sum())
            assert abs(di - kth) <= RTOL * max(abs(kth), 1e-30), \
                f"query {q}: id {i} differs from the oracle and is not a tie at the k-th distance"


def _filter_from(gpu, kind, n_base, density, seed):
    """(device filter or None, passing mask as uint8) for the filter layouts under test."""
    if kind == "none":
        return None, None
    rng = np.random.default_rng(seed)
    ids = np.nonzero(rng.random(n_base) < density)[0].astype(np.uint32)
    mask = np.zeros(n_base, np.uint8)
    mask[ids] = 1
    if kind == "ids":  # all-bitmap, universe = n_base (negated above 50%)
        g = gpu.upload_from_ids(ids, n_base)
    elif kind == "keep":  # array / bitmap containers
        lt = orc.Lite.from_sorted_ids(ids)
        g = gpu.upload_containers(lt.containers(), n_base, False, lt.cardinality(), orc.PROMOTE_KEEP_DEFAULT)
    elif kind == "runs":
        run_ids = np.concatenate([np.arange(s, min(n_base, s + 700)) for s in range(0, n_base, 2000)])
        run_ids = run_ids.astype(np.uint32)
        mask = np.zeros(n_base, np.uint8)
        mask[run_ids] = 1
        lt = orc.Lite.from_sorted_ids(run_ids).run_optimize()
        g = gpu.upload_containers(lt.containers(), 0, False, 0, orc.PROMOTE_KEEP_DEFAULT)
    elif kind == "setop":  # a set-operation result: no key_index, max_key 0 (found by key search)
        other = np.nonzero(rng.random(n_base) < 0.6)[0].astype(np.uint32)
        ga = gpu.upload_from_ids(ids, n_base)
        gb = gpu.upload_from_ids(other, n_base)
        g = gpu.set_operation(ga, gb, gpu.AND)
        gpu.free(ga)
        gpu.free(gb)
        assert not g.key_index
        mask = np.zeros(n_base, np.uint8)
        mask[np.intersect1d(ids, other)] = 1
    elif kind == "beyond":  # filter ids past n_base are ignored
        extra = np.arange(n_base, n_base + 5000, dtype=np.uint32)
        g = gpu.upload_from_ids(np.concatenate([ids, extra]), n_base + 70000)
    else:
        raise ValueError(kind)
    return g, mask


CASES = [
    # (n_base, n_q, dim, k, filter kind, density, seed)
    (5000, 40, 128, 10, "none", 1.0, 1),
    (5000, 40, 128, 100, "none", 1.0, 2),
    (20000, 300, 128, 10, "ids", 0.3, 3),
    (20000, 64, 128, 100, "ids", 0.7, 4),  # negated filter
    (150000, 33, 128, 100, "keep", 0.01, 5),
    (150000, 33, 128, 10, "keep", 0.4, 6),
    (140000, 20, 128, 50, "runs", 0.0, 7),
    (30000, 16, 128, 10, "beyond", 0.2, 8),
    (3000, 10, 64, 256, "none", 1.0, 9),
    (4000, 12, 100, 30, "ids", 0.5, 10),
    (4000, 12, 17, 30, "none", 1.0, 11),
    (2500, 7, 32, 10, "keep", 0.002, 12),  # fewer passing ids than k
    (70000, 520, 128, 10, "none", 1.0, 13),  # three query blocks
    (16384, 40, 128, 100, "none", 1.0, 14),  # the small-set limit exactly
    (16385, 40, 128, 100, "none", 1.0, 15),  # one row past it
    (3000, 9, 64, 10, "keep", 0.0, 16),  # no passing row: every slot is (+inf, -1)
    (60000, 20, 64, 10, "setop", 0.3, 17),
    (5000, 20, 17, 10, "keep", 0.3, 18),  # a filter with scalar row loads (dim % 4 != 0)
    (50000, 20, 72, 10, "ids", 0.4, 19),  # a filter, dim 72 of the 128-wide tiles
    (41000, 30, 128, 40, "setop", 0.5, 20),  # a filtered list path with a partial last tile in every chunk
]


SMALL_LIMITS = {"lists": 0, "small_16384": 16384, "small_default": 1 << 18}


@pytest.fixture(params=list(SMALL_LIMITS))
def path(request, gpu):
    """Runs a test with the small-set path off (every case on the per-chunk
    candidate lists), with a limit of 16384 passing rows (both sides of it in
    the cases below), and with the default limit (every case here keeps every
    estimate and selects per query)."""
    prev = gpu.topk_set_small_limit(SMALL_LIMITS[request.param])
    yield request.param
    gpu.topk_set_small_limit(prev)


@pytest.mark.parametrize("n_base,n_q,dim,k,kind,density,seed", CASES)
def test_topk_parity(gpu, path, n_base, n_q, dim, k, kind, density, seed):
    _say("topk", path, n_base, n_q, dim, k, kind, density, seed)
    base, queries = _data(n_base, n_q, dim, seed)
    filt, mask = _filter_from(gpu, kind, n_base, density, seed)
    got_d, got_i = _run(gpu, base, queries, k, filt)
    check_topk(base, queries, k, mask, got_d, got_i)
    if filt is not None:
        gpu.free(filt)


def test_topk_ties_break_by_id(gpu, path):
    """Duplicate base vectors tie exactly; the smaller id comes first."""
    _say("topk ties")
    rng = np.random.default_rng(21)
    uniq = rng.standard_normal((50, 128)).astype(np.float32)
    base = np.repeat(uniq, 40, axis=0)  # 2000 rows, each vector 40 times
    perm = rng.permutation(base.shape[0])
    base = np.ascontiguousarray(base[perm])
    queries = np.ascontiguousarray(uniq[:5] + 0.01 * rng.standard_normal((5, 128)).astype(np.float32))
    got_d, got_i = _run(gpu, base, queries, 60, None)
    check_topk(base, queries, 60, None, got_d, got_i)
    for q in range(5):
        for a in range(59):
            if got_d[q, a] == got_d[q, a + 1]:
                assert got_i[q, a] < got_i[q, a + 1]


def test_topk_multi_and_filter(gpu, path):
    """The workload's shape: filter = multi_and of three predicates."""
    _say("topk multi_and filter")
    n_base = 200000
    preds = [mt_bernoulli(60 + i, 0.5, n_base) for i in range(3)]
    gs = [gpu.upload_from_ids(p, n_base) for p in preds]
    f = gpu.multi_and(gs)
    mask = np.ones(n_base, np.uint8)
    for p in preds:
        m = np.zeros(n_base, np.uint8)
        m[p] = 1
        mask &= m
    base, queries = _data(n_base, 24, 128, 61)
    got_d, got_i = _run(gpu, base, queries, 10, f)
    check_topk(base, queries, 10, mask, got_d, got_i)
    for g in gs + [f]:
        gpu.free(g)


def test_topk_understated_cardinality(gpu):
    """The host leaves the list path out when a filter's recorded cardinality
    fits the small-set limit.  A caller-built struct whose total_cardinality
    understates its set (the library's own results record the exact count) then
    reaches tk_select with more rows than the limit, which takes every passing
    row as a candidate: the answer is still exact."""
    _say("topk understated cardinality")
    prev = gpu.topk_set_small_limit(16384)
    try:
        n_base = 60000
        ids = mt_bernoulli(71, 0.5, n_base)  # ~30000 passing rows, past the limit
        g = gpu.upload_from_ids(ids, n_base)
        true_card = g.total_cardinality
        assert true_card > 16384
        g.total_cardinality = 100
        mask = np.zeros(n_base, np.uint8)
        mask[ids] = 1
        base, queries = _data(n_base, 12, 64, 72)
        got_d, got_i = _run(gpu, base, queries, 20, g)
        check_topk(base, queries, 20, mask, got_d, got_i)
        g.total_cardinality = true_card
        gpu.free(g)
    finally:
        gpu.topk_set_small_limit(prev)


def test_topk_rejects_unsupported(gpu):
    _say("topk unsupported")
    torch = _torch()
    base = torch.zeros((10, 200), device="cuda")
    q = torch.zeros((2, 200), device="cuda")
    d = torch.empty((2, 5), device="cuda")
    i = torch.empty((2, 5), dtype=torch.int64, device="cuda")
    with pytest.raises(gpu.CrError):
        gpu.topk_filtered(base, q, 5, None, d, i)

"""GPU parity at the BASELINE configurations' own sizes, through the C ABI,
against the CPU oracle (bit-exact, strict layout) or a flat-bitset truth:

  configs[0]  U = 2^24: A 1% and B 10% uniform draws, the four operations
              with their cardinalities, 1M uniform point queries;
  configs[2]  U = 2^30, KEEP uploads: A/A' 0.1% (arrays), B/B' 50% (bitmaps),
              C/C' runs U[1k,64k) to 20% (run_optimize -> runs); the nine
              pairs x four operations; multi_and over 3 and 8 bitmaps drawn
              from {0.1, 1, 10, 50}%, pairwise (KEEP) and fused (ALL);
  configs[3]  U = 2^30 at 0.1/1/10/50%, compressed (KEEP) and promoted (ALL)
              layouts, uniform and sorted-clustered queries, every query mode;
  configs[4]  the filtered top-k at 10M x 128 with 1024 queries, k = 10 and
              100, every selectivity: 8 sampled queries against the fp64
              brute force (1e-4 relative, ids equal except at ties).

Inputs come from bench.py's generators, so these are the inputs the bench
times.  Each case prints what it runs before touching the GPU.
"""
import numpy as np
import pytest

import bench
import orc
from helpers import assert_packed_offsets, assert_same

pytestmark = pytest.mark.gpu

U = 1 << 30


def _say(*a):
    print("CASE", *a, flush=True)


@pytest.fixture(scope="module")
def torch():
    import torch as t
    return t


# ---- configs[0] ------------------------------------------------------------------------
def test_config0(gpu, torch):
    _say("configs[0] 2^24")
    U0 = 1 << 24
    a = np.random.default_rng(1).integers(0, U0, 167_772, dtype=np.uint64).astype(np.uint32)
    b = np.random.default_rng(2).integers(0, U0, 1_677_722, dtype=np.uint64).astype(np.uint32)
    q = np.random.default_rng(3).integers(0, U0, 1_000_000, dtype=np.uint64).astype(np.uint32)
    oa, ob = orc.upload_from_ids(a, U0), orc.upload_from_ids(b, U0)
    ga, gb = gpu.upload_from_ids(a, U0), gpu.upload_from_ids(b, U0)
    assert_same(gpu.download(ga), oa, strict=True, what="A")
    assert_same(gpu.download(gb), ob, strict=True, what="B")
    sa, sb = np.unique(a), np.unique(b)
    truth = {orc.AND: np.intersect1d(sa, sb).size, orc.OR: np.union1d(sa, sb).size,
             orc.ANDNOT: np.setdiff1d(sa, sb).size, orc.XOR: np.setxor1d(sa, sb).size}
    for op in (orc.AND, orc.OR, orc.ANDNOT, orc.XOR):
        r = gpu.set_operation(ga, gb, op)
        assert_same(gpu.download(r), orc.set_operation(oa, ob, op), strict=True, what=f"op {op}")
        assert gpu.cardinality(r) == truth[op]
        gpu.free(r)
    dq = torch.from_numpy(q.view(np.int32)).cuda()
    out = torch.empty_like(dq)
    for mode in (0, 1, 2, 3, 4):
        gpu.contains_batch(ga, dq, out, mode)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint32), np.isin(q, sa).astype(np.uint32))
    gpu.free(ga)
    gpu.free(gb)


# ---- configs[2] ------------------------------------------------------------------------
@pytest.fixture(scope="module")
def operands(gpu, torch):
    """{name: (oracle HostRoaring of the KEEP upload, GPU KEEP upload)}."""
    _say("configs[2] operands")
    out = {}
    for name, make in (("A", lambda: bench.words_bernoulli(torch, 0.001, 30)),
                       ("A'", lambda: bench.words_bernoulli(torch, 0.001, 31)),
                       ("B", lambda: bench.words_bernoulli(torch, 0.5, 32)),
                       ("B'", lambda: bench.words_bernoulli(torch, 0.5, 33)),
                       ("C", lambda: bench.words_runs(0.2, 34)), ("C'", lambda: bench.words_runs(0.2, 35))):
        lite = orc.Lite.from_words(make())
        if name.startswith("C"):
            lite.run_optimize()
        g = bench.keep_upload(gpu, lite)
        want = orc.upload_packed(lite, None, orc.PROMOTE_KEEP_DEFAULT)
        got = gpu.download(g)
        assert_same(got, want, strict=True, what=f"operand {name}")
        assert_packed_offsets(got, what=f"operand {name}")
        out[name] = (want, g)
    types = {k: (v[1].n_array_containers, v[1].n_bitmap_containers, v[1].n_run_containers) for k, v in out.items()}
    assert types["A"][0] > 0 and types["B"][1] > 0 and types["C"][2] > 0, types
    yield out
    for _, g in out.values():
        gpu.free(g)


@pytest.mark.parametrize("x,y", bench.SETOP_PAIRS)
def test_config2_set_operations(gpu, operands, x, y):
    (oa, ga), (ob, gb) = operands[x], operands[y]
    for op in (orc.AND, orc.OR, orc.ANDNOT, orc.XOR):
        _say("configs[2]", x, y, op)
        r = gpu.set_operation(ga, gb, op)
        assert_same(gpu.download(r), orc.set_operation(oa, ob, op), strict=True, what=f"{x}{y} op {op}")
        gpu.free(r)


@pytest.mark.parametrize("k,dens", [(3, (0.001, 0.1, 0.5)), (8, (0.001, 0.001, 0.01, 0.01, 0.1, 0.1, 0.5, 0.5))])
def test_config2_multi_and(gpu, torch, k, dens):
    lites = [orc.Lite.from_words(bench.words_bernoulli(torch, d, 100 + i)) for i, d in enumerate(dens)]
    for route, thr in (("pairwise", orc.PROMOTE_KEEP_DEFAULT), ("fused", orc.PROMOTE_ALL)):
        _say("configs[2] multi_and", k, route)
        gs = [gpu.upload_containers(lt.containers(), 0, False, 0, thr) for lt in lites]
        want = orc.multi_and([orc.upload_packed(lt, None, thr) for lt in lites])
        r = gpu.multi_and(gs)
        assert_same(gpu.download(r), want, strict=True, what=f"multi_and k={k} {route}")
        truth = lites[0]
        for lt in lites[1:]:
            truth = truth.op(lt, orc.AND)
        assert gpu.cardinality(r) == truth.cardinality()
        for g in gs + [r]:
            gpu.free(g)


# ---- configs[3] ------------------------------------------------------------------------
@pytest.fixture(scope="module")
def queries(gpu, torch):
    qs = bench.query_sets(torch)  # the bench's 100M uniform and 100M sorted-clustered queries
    yield qs
    del qs


@pytest.mark.parametrize("j,dens", list(enumerate((0.001, 0.01, 0.1, 0.5))))
def test_config3_point_queries(gpu, torch, queries, j, dens):
    """Every density, both layouts and both query sets against the flat
    bitset (one gather on the device): modes 0 (contains) and 4 (partitioned)
    on all 100M queries the bench times, modes 1-3 on the first 10M."""
    words = bench.words_bernoulli(torch, dens, 40 + j)
    lite = orc.Lite.from_words(words)
    w32 = torch.from_numpy(words.view(np.int32)).cuda()
    layouts = {"compressed": bench.keep_upload(gpu, lite),
               "promoted": gpu.upload_containers(lite.containers(), 0, False, 0, orc.PROMOTE_ALL)}
    if dens < 0.02:
        assert layouts["compressed"].n_array_containers > 0
    assert layouts["promoted"].n_array_containers == 0
    for qname, q in queries.items():
        q64 = q.to(torch.int64)
        truth = ((w32[q64 >> 5].to(torch.int64) >> (q64 & 31)) & 1).to(torch.int32)
        out = torch.empty_like(q)
        for lname, g in layouts.items():
            for mode in (0, 1, 2, 3, 4):
                nq = q.numel() if mode in (0, 4) else 10_000_000
                _say("configs[3]", dens, lname, qname, mode, nq)
                out.fill_(-1)
                gpu.contains_batch(g, q[:nq], out[:nq], mode)
                torch.cuda.synchronize()
                assert torch.equal(out[:nq], truth[:nq]), (dens, lname, qname, mode)
    for g in layouts.values():
        gpu.free(g)


# ---- the filtered top-k at full size ---------------------------------------
@pytest.fixture(scope="module")
def topk_data(gpu, torch):
    g = torch.Generator(device="cuda")
    g.manual_seed(50)
    base = torch.randn((bench.TK_N, bench.TK_DIM), device="cuda", dtype=torch.float32, generator=g)
    g.manual_seed(51)
    queries = torch.randn((bench.TK_Q, bench.TK_DIM), device="cuda", dtype=torch.float32, generator=g)
    preds = bench.zipf_predicates(torch, (0.001, 0.01, 0.1, 0.5))
    filters = {"unfiltered": (None, None)}
    for s, (masks, _) in preds.items():
        gs = [gpu.upload_from_device_ids(torch.nonzero(m).flatten().to(torch.int32), bench.TK_N) for m in masks]
        f = gpu.multi_and(gs)
        for x in gs:
            gpu.free(x)
        passing = (masks[0] & masks[1] & masks[2]).to(torch.uint8).cpu().numpy()
        filters[f"sel_{s:g}"] = (f, passing)
    del preds
    yield base, queries, base.cpu().numpy(), filters
    for f, _ in filters.values():
        if f is not None:
            gpu.free(f)


def _torch_topk_fp64(torch, base, queries, k, passing):
    """Every query's k smallest squared L2 distances over the passing rows, in
    fp64 by torch on the device (an fp64 GEMM per 1M-row chunk,
    |q|^2 + |x|^2 - 2 q.x, then a top-k per chunk and one over the chunks'
    candidates): (distances, ids), ascending."""
    q64 = queries.to(torch.float64)
    qn = (q64 * q64).sum(dim=1, keepdim=True)
    cand_d, cand_i = [], []
    step = 1 << 20
    for r0 in range(0, base.shape[0], step):
        x = base[r0:r0 + step].to(torch.float64)
        d = qn + (x * x).sum(dim=1)[None, :] - 2.0 * (q64 @ x.T)
        if passing is not None:
            d.masked_fill_(~passing[r0:r0 + step][None, :], float("inf"))
        kk = min(k, d.shape[1])
        v, i = torch.topk(d, kk, dim=1, largest=False)
        cand_d.append(v)
        cand_i.append(i + r0)
        del x, d
    d = torch.cat(cand_d, dim=1)
    i = torch.cat(cand_i, dim=1)
    v, j = torch.topk(d, k, dim=1, largest=False)
    return v, torch.gather(i, 1, j)


def _check_all_queries(torch, base, queries, k, passing, got_d, got_i):
    """All queries against the fp64 device reference: padding past the passing
    count, ids in range, unique and inside the filter, distances within 1e-4
    relative of their exact fp64 values and ascending, and every id that differs
    from the reference's a tie at the k-th distance (the unit tests' rule)."""
    from test_gpu_topk import RTOL
    n_pass = base.shape[0] if passing is None else int(passing.sum().item())
    valid = min(k, n_pass)
    assert bool((got_i[:, valid:] == -1).all()) and bool(torch.isinf(got_d[:, valid:]).all())
    gi, gd = got_i[:, :valid], got_d[:, :valid].to(torch.float64)
    assert bool(((gi >= 0) & (gi < base.shape[0])).all())
    srt = torch.sort(gi, dim=1).values
    assert bool((srt[:, 1:] != srt[:, :-1]).all()), "duplicate ids"
    if passing is not None:
        assert bool(passing[gi].all()), "an id outside the filter"
    exact = ((base[gi].to(torch.float64) - queries[:, None, :].to(torch.float64)) ** 2).sum(dim=2)
    assert bool(((gd - exact).abs() <= RTOL * exact.abs()).all()), "a distance off by more than 1e-4 relative"
    assert bool((gd[:, 1:] >= gd[:, :-1]).all()), "not ascending"
    want_d, want_i = _torch_topk_fp64(torch, base, queries, valid, passing)
    kth = want_d[:, -1:]
    # an id the kernel returned that the reference did not, or the reverse, must tie at the k-th distance
    in_want = (gi[:, :, None] == want_i[:, None, :]).any(dim=2)
    in_got = (want_i[:, :, None] == gi[:, None, :]).any(dim=2)
    tol = RTOL * kth.abs().clamp_min(1e-30)
    assert bool(((exact - kth).abs()[~in_want] <= tol.expand_as(exact)[~in_want]).all()), "an extra id is not a tie"
    assert bool(((want_d - kth).abs()[~in_got] <= tol.expand_as(want_d)[~in_got]).all()), "a missing id is not a tie"


@pytest.mark.parametrize("k", [10, 100])
@pytest.mark.parametrize("sel", ["unfiltered", "sel_0.001", "sel_0.01", "sel_0.1", "sel_0.5"])
def test_config4_topk_full_size(gpu, torch, topk_data, k, sel):
    """All 1024 queries run and all are checked against an fp64 top-k that torch
    computes on the device; 8 of them (spread over the batch) also against the
    oracle's fp64 brute force."""
    from test_gpu_topk import check_topk
    _say("configs[4] top-k", k, sel)
    base, queries, hbase, filters = topk_data
    f, passing = filters[sel]
    dist = torch.empty((bench.TK_Q, k), device="cuda", dtype=torch.float32)
    ids = torch.empty((bench.TK_Q, k), device="cuda", dtype=torch.int64)
    gpu.topk_filtered(base, queries, k, f, dist, ids)
    torch.cuda.synchronize()
    dev_pass = None if passing is None else torch.from_numpy(passing.astype(bool)).cuda()
    _check_all_queries(torch, base, queries, k, dev_pass, dist, ids)
    sample = np.array([0, 129, 258, 387, 516, 645, 774, 1023])
    hq = queries.cpu().numpy()[sample]
    check_topk(hbase, hq, k, passing, dist.cpu().numpy()[sample], ids.cpu().numpy()[sample])

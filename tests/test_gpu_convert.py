"""GPU parity of the conversions: decompress_to_bitset, enumerate_ids,
promote_to_bitmap, promote_auto and the deep copy, through the C-ABI.

Each GPU result is compared bit-exactly with the oracle applied to the very
structure the GPU call read (downloaded), and where the domain fixes the
answer, with numpy truth built from the input ids.  Output buffers are
pre-filled with a sentinel to show that no call writes past its bound.
"""
import numpy as np
import pytest

import orc
from gpu_inputs import KINDS, make_bitmap as _make
from helpers import assert_same, flat_from_ids, auto_l2

pytestmark = pytest.mark.gpu

SENT32 = 0x5A5A5A5A
SENT64 = -7


def _say(*a):
    print("CASE", *a, flush=True)


def _torch():
    import torch
    return torch


# ---- decompress_to_bitset ---------------------------------------------------------
@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("size", ["exact", "short", "long"])
def test_decompress_parity(gpu, kind, size):
    _say("decompress", kind, size)
    torch = _torch()
    g, stored = _make(gpu, kind)
    host = gpu.download(g)
    exact = (g.universe_size + 31) // 32
    n_words = {"exact": exact, "short": max(1, exact // 2 + 5), "long": exact + 4100}[size]
    buf = torch.full((n_words + 64,), SENT32, dtype=torch.int32, device="cuda")
    gpu.decompress_to_bitset(g, buf, n_words)
    gpu.synchronize()
    got = buf.cpu().numpy().view(np.uint32)
    assert np.all(got[n_words:] == SENT32), "write past n_words"
    want = orc.decompress(host, n_words)
    assert np.array_equal(got[:n_words], want)
    if stored is not None and size == "exact":
        truth = flat_from_ids(stored, g.universe_size)
        if g.negated:
            full, tail = g.universe_size // 32, g.universe_size % 32
            truth[:full] = ~truth[:full]
            if tail:
                truth[full] ^= np.uint32((1 << tail) - 1)
        assert np.array_equal(got[:n_words], truth)
    gpu.free(g)


@pytest.mark.parametrize("kind", ["ids_keep", "negated_odd_u", "empty"])
def test_decompress_alloc(gpu, kind):
    _say("decompress_alloc", kind)
    g, _ = _make(gpu, kind)
    host = gpu.download(g)
    ptr, n = gpu.decompress_to_bitset_alloc(g)
    assert n == (g.universe_size + 31) // 32
    gpu.synchronize()
    got = gpu._d2h(ptr, n, np.uint32)
    gpu.device_free(ptr)
    assert np.array_equal(got, orc.decompress(host, n))
    gpu.free(g)


def test_decompress_zero_universe(gpu):
    _say("decompress zero universe")
    g = gpu.GpuRoaring()
    ptr, n = gpu.decompress_to_bitset_alloc(g)
    assert ptr is None and n == 0
    gpu.decompress_to_bitset(g, _torch().zeros(1, dtype=_torch().int32, device="cuda"), 0)


# ---- enumerate_ids -------------------------------------------------------------------
@pytest.mark.parametrize("kind", KINDS)
def test_enumerate_parity(gpu, kind):
    _say("enumerate", kind)
    torch = _torch()
    g, stored = _make(gpu, kind)
    host = gpu.download(g)
    want = orc.enumerate_ids(host)
    if stored is not None and g.total_cardinality > 0:
        assert np.array_equal(want, stored.astype(np.int64))
    n = want.size
    buf = torch.full((n + 64,), SENT64, dtype=torch.int64, device="cuda")
    gpu.enumerate_ids(g, buf)
    gpu.synchronize()
    got = buf.cpu().numpy()
    assert np.array_equal(got[:n], want)
    assert np.all(got[n:] == SENT64), "write past the stored ids"
    if kind == "setop_result":  # total_cardinality is 0 on a set-op result: nothing is written
        assert g.total_cardinality == 0 and np.all(got == SENT64)
    gpu.free(g)


@pytest.mark.parametrize("kind", ["ids_keep", "runs_mixed", "arrays_only", "negated_odd_u"])
def test_enumerate_capacity_bound(gpu, kind):
    _say("enumerate capacity", kind)
    torch = _torch()
    g, _ = _make(gpu, kind)
    want = orc.enumerate_ids(gpu.download(g))
    cap = want.size // 2 + 3
    buf = torch.full((want.size + 8,), SENT64, dtype=torch.int64, device="cuda")
    gpu.enumerate_ids(g, buf, cap)
    gpu.synchronize()
    got = buf.cpu().numpy()
    assert np.array_equal(got[:cap], want[:cap])
    assert np.all(got[cap:] == SENT64)
    gpu.free(g)


@pytest.mark.parametrize("kind", ["ids_keep", "runs_mixed", "negated_runs", "setop_result", "empty"])
def test_enumerate_alloc(gpu, kind):
    _say("enumerate_alloc", kind)
    g, _ = _make(gpu, kind)
    want = orc.enumerate_ids(gpu.download(g))
    ptr, n = gpu.enumerate_ids_alloc(g)
    if g.total_cardinality == 0:
        assert ptr is None and n == 0
    else:
        assert n == want.size
        gpu.synchronize()
        got = gpu._d2h(ptr, n, np.int64)
        gpu.device_free(ptr)
        assert np.array_equal(got, want)
    gpu.free(g)


# ---- promote / deep copy ----------------------------------------------------------------
@pytest.mark.parametrize("kind", KINDS)
def test_promote_to_bitmap_parity(gpu, kind):
    _say("promote_to_bitmap", kind)
    g, _ = _make(gpu, kind)
    host = gpu.download(g)
    p = gpu.promote_to_bitmap(g)
    gpu.synchronize()
    want = orc.promote_to_bitmap(host)
    got = gpu.download(p)
    assert_same(got, want, strict=True, what="promote_to_bitmap")
    if g.n_containers:
        assert np.array_equal(orc.decompress(got), orc.decompress(host))
    gpu.free(p)
    gpu.free(g)


@pytest.mark.parametrize("kind", KINDS)
def test_deep_copy_parity(gpu, kind):
    _say("deep_copy", kind)
    g, _ = _make(gpu, kind)
    host = gpu.download(g)
    d = gpu.deep_copy(g)
    gpu.synchronize()
    want = orc.deep_copy(host)
    gpu.free(g)  # the copy owns independent memory
    assert_same(gpu.download(d), want, strict=True, what="deep_copy")
    gpu.free(d)


@pytest.mark.parametrize("universe", [1 << 22, 1 << 30])
def test_promote_auto_parity(gpu, universe):
    _say("promote_auto", universe)
    rng = np.random.default_rng(universe % 1000)
    ids = np.unique(rng.integers(0, universe, 3000, dtype=np.uint64).astype(np.uint32))
    g = gpu.upload_from_ids(ids, universe, orc.PROMOTE_KEEP_DEFAULT)
    host = gpu.download(g)
    p = gpu.promote_auto(g)
    gpu.synchronize()
    want = orc.promote_auto(host, auto_l2(gpu))
    assert_same(gpu.download(p), want, strict=True, what="promote_auto")
    if orc.resolve_auto_threshold(universe, auto_l2(gpu)) == orc.PROMOTE_ALL:
        assert p.n_array_containers == 0 and p.n_bitmap_containers == p.n_containers
    gpu.free(p)
    gpu.free(g)


# ---- size-independent properties at a large universe ------------------------------------------
def test_conversions_large_properties(gpu):
    """20M ids over 2^31: enumerate returns np.unique(ids); the bitset holds exactly
    those bits; promote -> enumerate gives the same ids."""
    _say("conversions large 20M / 2^31")
    torch = _torch()
    rng = np.random.default_rng(2024)
    U = 1 << 31
    ids = rng.integers(0, U, 20_000_000, dtype=np.uint64).astype(np.uint32)
    want = np.unique(ids)
    g = gpu.upload_from_ids(ids, U, orc.PROMOTE_KEEP_DEFAULT)
    out = torch.empty(want.size, dtype=torch.int64, device="cuda")
    gpu.enumerate_ids(g, out)
    gpu.synchronize()
    assert np.array_equal(out.cpu().numpy(), want.astype(np.int64))
    del out
    words = torch.empty(U // 32, dtype=torch.int32, device="cuda")
    gpu.decompress_to_bitset(g, words)
    gpu.synchronize()
    flat = words.cpu().numpy().view(np.uint32)
    del words
    assert int(np.bitwise_count(flat).sum(dtype=np.uint64)) == want.size
    assert np.all((flat[want >> 5] >> (want & 31)) & 1)
    p = gpu.promote_to_bitmap(g)
    out = torch.empty(want.size, dtype=torch.int64, device="cuda")
    gpu.enumerate_ids(p, out)
    gpu.synchronize()
    assert np.array_equal(out.cpu().numpy(), want.astype(np.int64))
    gpu.free(p)
    gpu.free(g)


# ---- cardinality ---------------------------------------------------------------------
@pytest.mark.parametrize("kind", KINDS)
def test_cardinality(gpu, kind):
    """The device count equals the popcount of the oracle's logical decode of the
    same structure (set-operation results, whose total_cardinality is 0, included)."""
    _say("cardinality", kind)
    g, stored = _make(gpu, kind)
    host = gpu.download(g)
    want = int(np.bitwise_count(orc.decompress(host)).sum()) if host.universe_size else orc.true_cardinality(host)
    if stored is not None and not g.negated:
        assert want == stored.size
    assert gpu.cardinality(g) == want
    gpu.free(g)

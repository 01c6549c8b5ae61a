"""cr_enumerate_ids_noalloc -- enumerate_ids with no device allocation (its
scratch is the library's fixed per-device array) -- against cr_enumerate_ids
on the same bitmaps, bit-exact, through the C ABI.  Calls come in a row, each
later one on a smaller input, so counts or starts left in the shared scratch by
an earlier call would show up as wrong ids."""
import numpy as np
import pytest

import orc
from gpu_inputs import KINDS, make_bitmap

pytestmark = pytest.mark.gpu
SENT64 = -7777


def _say(*a):
    print("CASE", *a, flush=True)


def _stored(g):
    if g.total_cardinality == 0:
        return 0
    return g.universe_size - g.total_cardinality if g.negated else g.total_cardinality


def _both(gpu, g):
    """(existing entry point's output, no-alloc output), each with 64 sentinel slots past the end."""
    import torch
    n = _stored(g)
    a = torch.full((n + 64,), SENT64, dtype=torch.int64, device="cuda")
    b = torch.full((n + 64,), SENT64, dtype=torch.int64, device="cuda")
    gpu.enumerate_ids(g, a)
    gpu.enumerate_ids_noalloc(g, b)
    gpu.synchronize()
    return a.cpu().numpy(), b.cpu().numpy(), n


def test_noalloc_matches_enumerate_ids_large_then_small(gpu):
    rng = np.random.default_rng(5)
    U = 1 << 30
    big_ids = rng.integers(0, U, 3_000_000, dtype=np.uint64).astype(np.uint32)
    small_ids = rng.integers(0, 1 << 22, 50_000, dtype=np.uint64).astype(np.uint32)
    for what, ids, u in (("16384 bitmaps over 2^30", big_ids, U), ("64 bitmaps over 2^22", small_ids, 1 << 22)):
        _say("enumerate_ids_noalloc", what)
        g = gpu.upload_from_ids(ids, u)
        want, got, n = _both(gpu, g)
        assert n == np.unique(ids).size
        assert np.array_equal(got, want)
        assert np.array_equal(got[:n], np.unique(ids).astype(np.int64))
        assert np.all(got[n:] == SENT64)
        gpu.free(g)


def test_noalloc_matches_enumerate_ids_every_layout(gpu):
    """Every bitmap shape in a row (arrays, runs, negated, empty, set-operation results)."""
    for kind in KINDS:
        _say("enumerate_ids_noalloc", kind)
        g, _ = make_bitmap(gpu, kind)
        want, got, n = _both(gpu, g)
        assert np.array_equal(got, want), kind
        assert np.array_equal(got[:n], orc.enumerate_ids(gpu.download(g))), kind
        gpu.free(g)


def test_noalloc_capacity_bound(gpu):
    import torch
    _say("enumerate_ids_noalloc capacity")
    g, _ = make_bitmap(gpu, "runs_mixed")
    n = _stored(g)
    cap = n // 3 + 1
    a = torch.full((n + 8,), SENT64, dtype=torch.int64, device="cuda")
    b = torch.full((n + 8,), SENT64, dtype=torch.int64, device="cuda")
    gpu.enumerate_ids(g, a, cap)
    gpu.enumerate_ids_noalloc(g, b, cap)
    gpu.synchronize()
    assert np.array_equal(a.cpu().numpy(), b.cpu().numpy())
    assert np.all(b.cpu().numpy()[cap:] == SENT64)
    gpu.free(g)


def test_noalloc_rejects_more_containers_than_its_scratch(gpu):
    """Checked on the host before any launch: the struct's pointers are never read."""
    import torch
    _say("enumerate_ids_noalloc rejection")
    g = gpu.GpuRoaring()
    g.n_containers = 65537
    g.total_cardinality = 1
    out = torch.zeros(8, dtype=torch.int64, device="cuda")
    with pytest.raises(gpu.CrError, match="scratch bound"):
        gpu.enumerate_ids_noalloc(g, out)

"""GPU parity of the batch API (the reference's v2) through the C-ABI.

Every device result is downloaded and compared field by field with the batch
oracle (oracle/batch.py) on the same inputs: CSR starts, keys, types,
offsets, cardinalities, key indices, pools and the host mirrors, bit-exact.
Queries and decompress are compared on the same ids / buffers.
"""
import numpy as np
import pytest

import batch as ob
import orc
from test_oracle_batch import PROBES, _random_lites, mixed_lite

pytestmark = pytest.mark.gpu

FIELDS = ("container_starts", "key_index_starts", "keys", "types", "offsets", "cards", "key_indices",
          "bitmap_data", "array_data", "run_data", "host_total_cardinalities", "host_universe_sizes",
          "host_container_starts", "host_key_index_starts", "host_n_bitmap_containers")


def _say(*a):
    print("CASE", *a, flush=True)


def _torch():
    import torch
    return torch


def assert_batch(got, want, what=""):
    for k in ("n_bitmaps", "total_containers", "n_bitmap_containers_total", "array_pool_bytes", "run_pool_bytes"):
        assert int(getattr(got, k)) == int(getattr(want, k)), f"{what}: {k} {getattr(got, k)} != {getattr(want, k)}"
    for f in FIELDS:
        g, w = np.asarray(getattr(got, f)), np.asarray(getattr(want, f))
        assert g.size == w.size and np.array_equal(g.astype(w.dtype), w), f"{what}: field {f} differs"


def _inputs(seed):
    rng = np.random.default_rng(seed)
    lites, _ = _random_lites(rng, 7)
    lites.insert(3, orc.Lite.from_sorted_ids(np.zeros(0, np.uint32)))  # an empty bitmap inside the batch
    lites += [mixed_lite(v) for v in range(4)]
    return lites


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_upload_and_promote_parity(gpu, seed):
    _say("upload_batch / promote_batch", seed)
    lites = _inputs(seed)
    conts = [l.containers() for l in lites]
    want = ob.upload_batch(conts)
    B = gpu.upload_batch(conts)
    assert_batch(gpu.download_batch(B), want, "upload_batch")
    P = gpu.promote_batch(B)
    gpu.synchronize()
    assert_batch(gpu.download_batch(P), ob.promote_batch(want), "promote_batch")
    gpu.free_batch(P)
    gpu.free_batch(B)


def test_empty_batch(gpu):
    _say("empty batch")
    B = gpu.upload_batch([])
    assert B.n_bitmaps == 0 and not B._alloc_base
    P = gpu.promote_batch(B)
    assert P.n_bitmaps == 0
    gpu.batch_decompress(B, _torch().zeros(1, dtype=_torch().int64, device="cuda"), 0)
    gpu.free_batch(B)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_multi_and_parity(gpu, seed):
    _say("batch multi_and", seed)
    lites = _inputs(seed)
    conts = [l.containers() for l in lites]
    hb = ob.promote_batch(ob.upload_batch(conts))
    B = gpu.upload_batch(conts)
    P = gpu.promote_batch(B)
    rng = np.random.default_rng(seed + 10)
    sets = [[0], [8, 9, 10], [9, 10, 11], [8, 9, 10, 11], [0, 1, 2, 4, 5], [2, 2, 5], [3, 5], list(range(12))]
    sets += [list(rng.choice(12, int(rng.integers(2, 6)), replace=True)) for _ in range(4)]
    sets += [list(range(12)) * 6, [9] * 64, [9] * 65]  # both sides of the 64-input wavefront path
    for idx in sets:
        want = ob.multi_and(hb, idx)
        R = gpu.batch_multi_and(P, idx)
        assert_batch(gpu.download_batch(R), want, f"multi_and {idx}")
        gpu.free_batch(R)
    # the raw batch holds array / run containers; bad index; no inputs
    with pytest.raises(gpu.CrError) as e:
        gpu.batch_multi_and(B, [8, 9])
    assert e.value.code == gpu.CR_ERR_INVALID
    with pytest.raises(gpu.CrError) as e:
        gpu.batch_multi_and(P, [0, 12])
    assert e.value.code == gpu.CR_ERR_RANGE
    with pytest.raises(gpu.CrError) as e:
        gpu.batch_multi_and(P, [])
    assert e.value.code == gpu.CR_ERR_INVALID
    gpu.free_batch(P)
    gpu.free_batch(B)


@pytest.mark.parametrize("seed", [0, 1])
def test_decompress_parity(gpu, seed):
    _say("decompress_batch", seed)
    torch = _torch()
    lites = _inputs(seed)
    conts = [l.containers() for l in lites]
    hb = ob.upload_batch(conts)
    B = gpu.upload_batch(conts)
    need = (int(hb.host_universe_sizes.max()) + 63) // 64
    for words_each, fill in ((need, 0), (need + 37, 0), (need, 0x8000000000000001)):
        prior = np.full(B.n_bitmaps * words_each, np.uint64(fill), np.uint64)
        d = torch.from_numpy(prior.view(np.int64).copy()).cuda()
        gpu.batch_decompress(B, d, words_each)
        gpu.synchronize()
        got = d.cpu().numpy().view(np.uint64)
        assert np.array_equal(got, ob.decompress_batch(hb, words_each, prior)), (words_each, fill)
    with pytest.raises(gpu.CrError) as e:
        gpu.batch_decompress(B, torch.zeros(B.n_bitmaps * need, dtype=torch.int64, device="cuda"), need - 1)
    assert e.value.code == gpu.CR_ERR_INVALID
    gpu.free_batch(B)


@pytest.mark.parametrize("promoted", [False, True])
def test_contains_parity(gpu, promoted):
    _say("batch contains", promoted)
    torch = _torch()
    lites = _inputs(5)
    conts = [l.containers() for l in lites]
    hb = ob.upload_batch(conts)
    B = gpu.upload_batch(conts)
    if promoted:
        hb, B = ob.promote_batch(hb), gpu.promote_batch(B)
    rng = np.random.default_rng(3)
    ids = np.concatenate([PROBES, rng.integers(0, 14 * 65536, 4000).astype(np.uint32),
                          np.array([0, 65535, 65536, 0xFFFFFFFF], np.uint32)])
    d_ids = torch.from_numpy(ids.view(np.int32).copy()).cuda()
    out = torch.empty(ids.size, dtype=torch.uint8, device="cuda")
    for b in range(hb.n_bitmaps + 1):  # b == n_bitmaps answers false
        gpu.batch_contains(B, d_ids, out, bitmap=b)
        gpu.synchronize()
        assert np.array_equal(out.cpu().numpy(), ob.contains(hb, b, ids)), b
        if b < hb.n_bitmaps:
            v = gpu.batch_make_view(B, b)
            gpu.batch_view_contains(v, d_ids, out)
            gpu.synchronize()
            assert np.array_equal(out.cpu().numpy(), ob.view_contains(hb, b, ids)), b
    # per-query bitmap index: the multi-filter shape
    bidx = rng.integers(0, hb.n_bitmaps, ids.size).astype(np.uint32)
    d_b = torch.from_numpy(bidx.view(np.int32).copy()).cuda()
    gpu.batch_contains(B, d_ids, out, d_bitmap_idx=d_b)
    gpu.synchronize()
    want = np.array([ob.contains(hb, int(b), ids[i:i + 1])[0] for i, b in enumerate(bidx)], np.uint8)
    assert np.array_equal(out.cpu().numpy(), want)
    with pytest.raises(gpu.CrError) as e:
        gpu.batch_make_view(B, hb.n_bitmaps)
    assert e.value.code == gpu.CR_ERR_RANGE
    gpu.free_batch(B)


def test_reference_n4_flow(gpu):
    """v2/test/test_basic.cu:208-420 on the GPU: cardinalities, contains, promote
    invariants, multi_and {0,1,2} / {2,3} against roaring-lite AND, decompress."""
    _say("v2 reference n=4 flow")
    torch = _torch()
    lites = [mixed_lite(v) for v in range(4)]
    B = gpu.upload_batch([l.containers() for l in lites])
    hb = gpu.download_batch(B)
    d_ids = torch.from_numpy(PROBES.view(np.int32).copy()).cuda()
    out = torch.empty(PROBES.size, dtype=torch.uint8, device="cuda")
    for b, l in enumerate(lites):
        assert int(hb.host_total_cardinalities[b]) == l.cardinality()
        gpu.batch_contains(B, d_ids, out, bitmap=b)
        gpu.synchronize()
        assert np.array_equal(out.cpu().numpy(), l.contains_many(PROBES).astype(np.uint8))
    P = gpu.promote_batch(B)
    gpu.synchronize()
    assert P.n_bitmap_containers_total == P.total_containers == B.total_containers
    for idx in ([0, 1, 2], [2, 3]):
        exp = lites[idx[0]]
        for j in idx[1:]:
            exp = exp.op(lites[j], orc.AND)
        R = gpu.batch_multi_and(P, idx)
        assert int(R.host_total_cardinalities[0]) == exp.cardinality()
        gpu.batch_contains(R, d_ids, out, bitmap=0)
        gpu.synchronize()
        assert np.array_equal(out.cpu().numpy(), exp.contains_many(PROBES).astype(np.uint8))
        gpu.free_batch(R)
    gpu.free_batch(P)
    gpu.free_batch(B)


def test_large_batch_properties(gpu):
    """64 bitmaps over 2^24 (mixed containers), multi_and of 8: the result equals
    numpy's intersection; decompress of every bitmap equals its id set."""
    _say("large batch 64 x 2^24")
    torch = _torch()
    rng = np.random.default_rng(99)
    U = 1 << 24
    sets = []
    base_dense = np.nonzero(rng.random(U) < 0.5)[0]
    for b in range(64):
        keep = rng.random(base_dense.size) < 0.9
        extra = np.unique(rng.integers(0, U, 20000))
        sets.append(np.unique(np.concatenate([base_dense[keep], extra])).astype(np.uint32))
    lites = [orc.Lite.from_sorted_ids(s).run_optimize() for s in sets]
    B = gpu.upload_batch([l.containers() for l in lites])
    P = gpu.promote_batch(B)
    idx = list(range(0, 64, 8))
    R = gpu.batch_multi_and(P, idx)
    inter = sets[idx[0]]
    for j in idx[1:]:
        inter = np.intersect1d(inter, sets[j], assume_unique=True)
    assert int(R.host_total_cardinalities[0]) == inter.size
    words_each = U // 64
    d = torch.zeros(64 * words_each, dtype=torch.int64, device="cuda")
    gpu.batch_decompress(B, d, words_each)
    gpu.synchronize()
    flat = d.cpu().numpy().view(np.uint64).reshape(64, words_each)
    for b in (0, 17, 63):
        bits = np.unpackbits(flat[b].view(np.uint8), bitorder="little")
        assert np.array_equal(np.nonzero(bits)[0], sets[b])
    for x in (R, P, B):
        gpu.free_batch(x)

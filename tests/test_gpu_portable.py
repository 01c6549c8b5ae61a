"""GPU parity of the Roaring portable format through the C-ABI.

serialize: the GPU bytes equal the oracle writer's bytes for the bitmap's
logical set after run_optimize (the logical set is decoded by the oracle
from the structure the GPU read, so a negated bitmap is complemented within
U).  deserialize: the GPU result equals the oracle's packed upload of the
oracle reader's bitmap, with and without a universe (the latter decides the
complement, as upload(bm, U) does).
"""
import numpy as np
import pytest

import orc
from gpu_inputs import KINDS, make_bitmap
from helpers import assert_same, ids_from_flat, auto_l2

pytestmark = pytest.mark.gpu


def _say(*a):
    print("CASE", *a, flush=True)


def _logical_ids(host):
    if host.universe_size == 0:
        return np.zeros(0, np.uint32)
    return ids_from_flat(orc.decompress(host))


@pytest.mark.parametrize("kind", KINDS + ["promoted_runs"])
def test_serialize_parity(gpu, kind):
    _say("portable_serialize", kind)
    if kind == "promoted_runs":
        src, _ = make_bitmap(gpu, "runs_mixed")
        g = gpu.promote_to_bitmap(src)
        gpu.synchronize()
        gpu.free(src)
    else:
        g, _ = make_bitmap(gpu, kind)
    host = gpu.download(g)
    ids = _logical_ids(host)
    want = orc.Lite.from_sorted_ids(ids).run_optimize().portable_serialize()
    assert gpu.portable_size_in_bytes(g) == len(want)
    got = gpu.portable_serialize(g)
    assert got == want
    back = orc.Lite.portable_deserialize(got)
    assert np.array_equal(back.to_ids(), ids)
    gpu.free(g)


def _lites():
    rng = np.random.default_rng(77)
    U = 12 * 65536 + 300
    from gpu_inputs import run_heavy_ids
    runs = run_heavy_ids(rng, 8 * 65536)
    sparse = np.unique(rng.integers(0, U, 3000, dtype=np.uint64)).astype(np.uint32)
    dense = np.nonzero(rng.random(U) < 0.8)[0].astype(np.uint32)
    return U, {"runs": orc.Lite.from_sorted_ids(runs).run_optimize(),
               "sparse": orc.Lite.from_sorted_ids(sparse),
               "dense_runs": orc.Lite.from_sorted_ids(dense).run_optimize(),
               "empty": orc.Lite.from_sorted_ids(np.zeros(0, np.uint32))}


@pytest.mark.parametrize("name", ["runs", "sparse", "dense_runs", "empty"])
@pytest.mark.parametrize("with_u", [False, True])
@pytest.mark.parametrize("thr", [orc.PROMOTE_KEEP_DEFAULT, orc.PROMOTE_ALL])
def test_deserialize_parity(gpu, name, with_u, thr):
    _say("portable_deserialize", name, with_u, thr)
    U, lites = _lites()
    data = lites[name].portable_serialize()
    lite = orc.Lite.portable_deserialize(data)
    want = orc.upload_packed(lite, U if with_u else None, thr, auto_l2(gpu))
    g = gpu.portable_deserialize(data, U if with_u else 0, thr)
    assert_same(gpu.download(g), want, strict=True, what="portable_deserialize")
    # and back: the GPU writer gives the run-optimized bytes of the same logical
    # set, also when the upload stored the complement (negated)
    again = gpu.portable_serialize(g)
    assert again == orc.Lite.from_sorted_ids(lite.to_ids()).run_optimize().portable_serialize()
    gpu.free(g)


def test_serialize_capacity_error(gpu):
    _say("portable_serialize capacity")
    import ctypes as C
    g, _ = make_bitmap(gpu, "runs_mixed")
    n = gpu.portable_size_in_bytes(g)
    buf = C.create_string_buffer(n)
    w = C.c_size_t()
    rc = gpu.load().cr_portable_serialize(C.byref(g), None, buf, n - 1, C.byref(w))
    assert rc == gpu.CR_ERR_INVALID and w.value == n
    gpu.free(g)


def test_round_trip_large(gpu):
    """2^28 universe, dense, sparse and run keys: GPU serialize -> GPU deserialize
    -> GPU serialize is a fixed point and decodes to the input ids."""
    _say("portable round trip 2^28")
    rng = np.random.default_rng(5)
    U = 1 << 28
    parts = []
    for j, key in enumerate(range(0, U >> 16, 3)):
        base = key * 65536
        k = j % 3
        if k == 0:
            parts.append(base + np.nonzero(rng.random(65536) < 0.3)[0])
        elif k == 1:
            parts.append(base + np.unique(rng.integers(0, 65536, 200)))
        else:
            s = int(rng.integers(0, 30000))
            parts.append(base + np.arange(s, s + 20000))
    ids = np.unique(np.concatenate(parts)).astype(np.uint32)
    g = gpu.upload_from_ids(ids, U, orc.PROMOTE_KEEP_DEFAULT)
    data = gpu.portable_serialize(g)
    want = orc.Lite.from_sorted_ids(ids).run_optimize().portable_serialize()
    assert data == want
    h = gpu.portable_deserialize(data, U)
    assert gpu.portable_serialize(h) == data
    gpu.free(g)
    gpu.free(h)

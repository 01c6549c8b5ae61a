"""GPU tests of malformed inputs and of the error contract.

- set_operation on structs whose key_index does not describe their `keys`
  (an extra key, two entries swapped, an entry moved to an absent key): the
  reference matches containers on `keys` (src/set_ops.cu:76-122) and never
  reads key_index there, so the result must be the oracle's on the keys, both
  through the classify plan (mixed container types) and the all-bitmap plan;
- contains on a view that says all_bitmap but has no key_index: the reference
  takes its fast path only with a key_index (roaring_view.cuh:45), so every
  query mode must answer through the general lookup;
- device allocation failures, injected with cr_debug_fail_device_allocs, come
  back as CR_ERR_ALLOC from every producing call, leave the output struct
  empty, and leave the library working (the reference's contract is a thrown
  std::runtime_error, include/cu_roaring/detail/utils.cuh:9-18; the C++ side of
  it is checked in tests/cpp/api_check.cpp).
"""
import ctypes as C

import numpy as np
import pytest

import orc
from helpers import assert_same, auto_l2

pytestmark = pytest.mark.gpu


def _say(*a):
    print("CASE", *a, flush=True)


def _torch():
    import torch
    return torch


def _dev_u32(a):
    return _torch().from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).cuda()


def _with_key_index(gpu, g, kidx):
    """A copy of g's struct (aliasing g's device block) whose key_index is a new
    device array holding `kidx`; returns (struct, device pointer to free)."""
    lib = gpu.load()
    p = C.c_void_p()
    assert lib.cr_device_malloc(C.byref(p), kidx.nbytes) == 0
    assert lib.cr_memcpy_h2d(p, kidx.ctypes.data, kidx.nbytes) == 0
    x = gpu.GpuRoaring.from_buffer_copy(g)
    x.key_index = p.value
    return x, p


def _corruptions(kidx, keys, rng):
    """key_index variants that do not describe `keys`: an absent key named, two
    present entries swapped, a present entry moved to an absent key."""
    absent = np.nonzero(kidx == 0xFFFF)[0]
    present = np.nonzero(kidx != 0xFFFF)[0]
    assert absent.size and present.size >= 2
    out = {}
    x = kidx.copy()
    x[absent[0]] = 0
    out["extra_key"] = x
    x = kidx.copy()
    i, j = rng.choice(present, 2, replace=False)
    x[i], x[j] = x[j], x[i]
    out["swapped"] = x
    x = kidx.copy()
    k = rng.choice(present)
    x[absent[-1]] = x[k]
    x[k] = 0xFFFF
    out["moved"] = x
    return out


def _mixed_operands(seed):
    rng = np.random.default_rng(seed)
    U = 16 * 65536
    parts = [[], []]
    for key in range(16):
        for s in (0, 1):
            kind = rng.integers(0, 4)
            base = key * 65536
            if kind == 1:
                parts[s].append(base + np.unique(rng.integers(0, 65536, int(rng.integers(1, 3000)))))
            elif kind == 2:
                parts[s].append(base + np.nonzero(rng.random(65536) < 0.4)[0])
            elif kind == 3:
                st = int(rng.integers(0, 30000))
                parts[s].append(base + np.arange(st, st + int(rng.integers(100, 30000))))
    lites = [orc.Lite.from_sorted_ids(np.unique(np.concatenate(p)).astype(np.uint32)).run_optimize() for p in parts]
    return U, lites


@pytest.mark.parametrize("op", [orc.AND, orc.OR, orc.ANDNOT, orc.XOR])
@pytest.mark.parametrize("layout", ["mixed_types", "all_bitmap"])
def test_set_operation_inconsistent_key_index(gpu, op, layout):
    _say("set_operation inconsistent key_index", layout, op)
    rng = np.random.default_rng(11 + op)
    if layout == "mixed_types":
        U, (la, lb) = _mixed_operands(3)
        ga = gpu.upload_containers(la.containers(), 0, False, 0, orc.PROMOTE_KEEP_DEFAULT)
        gb = gpu.upload_containers(lb.containers(), 0, False, 0, orc.PROMOTE_KEEP_DEFAULT)
        oa = orc.upload_packed(la, None, orc.PROMOTE_KEEP_DEFAULT, auto_l2(gpu))
        ob = orc.upload_packed(lb, None, orc.PROMOTE_KEEP_DEFAULT, auto_l2(gpu))
        assert ga.n_array_containers + ga.n_run_containers > 0
    else:
        # every other key present: all-bitmap uploads that are not dense
        U = 40 * 65536
        ids = [np.nonzero(rng.random(U) < d)[0].astype(np.uint32) for d in (0.3, 0.5)]
        ids = [x[((x >> 16) % 3) != s] for x, s in zip(ids, (0, 1))]
        ga, gb = (gpu.upload_from_device_ids(_dev_u32(x), U) for x in ids)
        oa, ob = (orc.upload_from_ids(x, U) for x in ids)
        assert ga.n_array_containers == ga.n_run_containers == 0 and ga.n_containers < ga.max_key + 1
    assert ga.key_index and gb.key_index
    want = orc.set_operation(oa, ob, op)
    g = gpu.set_operation(ga, gb, op)  # the consistent inputs first
    assert_same(gpu.download(g), want, strict=True, what="consistent")
    gpu.free(g)
    kidx = gpu._d2h(ga.key_index, ga.max_key + 1, np.uint16)
    keys = gpu._d2h(ga.keys, ga.n_containers, np.uint16)
    for name, bad in _corruptions(kidx, keys, rng).items():
        _say("  corruption", name)
        x, p = _with_key_index(gpu, ga, bad)
        try:
            g = gpu.set_operation(x, gb, op)
            assert_same(gpu.download(g), want, strict=True, what=f"{layout} {name} (a)")
            gpu.free(g)
            g = gpu.set_operation(gb, x, op)
            assert_same(gpu.download(g), orc.set_operation(ob, oa, op), strict=True, what=f"{layout} {name} (b)")
            gpu.free(g)
        finally:
            gpu.device_free(p.value)
    gpu.free(ga)
    gpu.free(gb)


def test_contains_all_bitmap_view_without_key_index(gpu):
    """A hand-built view with all_bitmap set and no key_index answers through
    the key search in every mode."""
    _say("contains all_bitmap without key_index")
    torch = _torch()
    rng = np.random.default_rng(21)
    U = 24 * 65536
    ids = np.nonzero(rng.random(U) < 0.2)[0].astype(np.uint32)
    ids = ids[((ids >> 16) % 4) != 1]
    o = orc.upload_from_ids(ids, U)
    g = gpu.upload_from_device_ids(_dev_u32(ids), U)
    v = gpu.make_view(g)
    assert v.all_bitmap
    v.key_index = None
    v.all_bitmap = True
    q = rng.integers(0, U + 4 * 65536, 200000, dtype=np.uint64).astype(np.uint32)
    dq = _dev_u32(q)
    out = torch.empty_like(dq)
    want = orc.contains_many(o, q)
    lib = gpu.load()
    for mode in range(5):
        out.fill_(7)
        rc = lib.cr_contains_batch(C.byref(v), dq.data_ptr(), q.size, out.data_ptr(), mode, None)
        assert rc == 0, lib.cr_last_error()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want), f"mode {mode}"
    gpu.free(g)


def _calls(gpu):
    """(name, fn) for producing calls; each fn returns the C status and the output struct."""
    torch = _torch()
    lib = gpu.load()
    rng = np.random.default_rng(31)
    U = 1 << 26
    big = rng.integers(0, U, 3_000_000, dtype=np.uint64).astype(np.uint32)
    small = rng.integers(0, U, 700, dtype=np.uint64).astype(np.uint32)
    d_big, d_small = _dev_u32(big), _dev_u32(small)
    words = np.zeros(U // 32, np.uint32)
    np.bitwise_or.at(words, big[:200000] >> 5, np.uint32(1) << (big[:200000] & 31))
    d_words = _dev_u32(words)
    la = orc.Lite.from_sorted_ids(np.unique(big[:50000])).run_optimize()
    A = gpu.upload_from_device_ids(d_big, U)
    B = gpu.upload_containers(la.containers(), 0, False, 0, orc.PROMOTE_KEEP_DEFAULT)
    conts, conts_payloads = gpu._container_array(la.containers())
    n_conts = len(la.containers())
    keep = [d_big, d_small, d_words, conts, conts_payloads]

    def run(f):
        out = gpu.GpuRoaring()
        return f(out), out

    calls = [
        ("upload_from_device_ids", lambda: run(lambda o: lib.cr_upload_from_device_ids(
            d_big.data_ptr(), big.size, U, None, orc.PROMOTE_AUTO, C.byref(o)))),
        ("upload_from_device_ids_small", lambda: run(lambda o: lib.cr_upload_from_device_ids(
            d_small.data_ptr(), small.size, U, None, orc.PROMOTE_KEEP_DEFAULT, C.byref(o)))),
        ("upload_from_device_bitset", lambda: run(lambda o: lib.cr_upload_from_device_bitset(
            d_words.data_ptr(), words.size, U, None, C.byref(o)))),
        ("upload_containers", lambda: run(lambda o: lib.cr_upload_containers(
            conts, n_conts, 0, False, 0, None, orc.PROMOTE_KEEP_DEFAULT, C.byref(o)))),
        ("set_operation_dense", lambda: run(lambda o: lib.cr_set_operation(C.byref(A), C.byref(A), orc.XOR, None,
                                                                            C.byref(o)))),
        ("set_operation_mixed", lambda: run(lambda o: lib.cr_set_operation(C.byref(A), C.byref(B), orc.OR, None,
                                                                            C.byref(o)))),
        ("multi_and_fused", lambda: run(lambda o: lib.cr_multi_and((gpu.GpuRoaring * 2)(A, A), 2, None,
                                                                   C.byref(o)))),
        ("multi_and_pairwise", lambda: run(lambda o: lib.cr_multi_and((gpu.GpuRoaring * 2)(A, B), 2, None,
                                                                      C.byref(o)))),
        ("promote_to_bitmap", lambda: run(lambda o: lib.cr_promote_to_bitmap(C.byref(B), None, C.byref(o)))),
        ("deep_copy", lambda: run(lambda o: lib.cr_deep_copy(C.byref(B), None, C.byref(o)))),
    ]
    return calls, (A, B), keep


def test_alloc_failure_returns_cr_err_alloc(gpu):
    """For every producing call, failing its first, second, ... device
    allocation returns CR_ERR_ALLOC with an empty output struct, until the call
    makes fewer allocations than the skip; then it succeeds, and its result
    equals the one made without any injection."""
    lib = gpu.load()
    calls, owned, keep = _calls(gpu)
    try:
        for name, fn in calls:
            _say("alloc failure", name)
            rc, ref = fn()
            assert rc == 0, (name, lib.cr_last_error())
            gpu.synchronize()
            want = gpu.download(ref)
            gpu.free(ref)
            failures = 0
            for skip in range(16):
                lib.cr_debug_fail_device_allocs(skip, 1)
                rc, out = fn()
                lib.cr_debug_fail_device_allocs(0, 0)
                if rc == 0:
                    gpu.synchronize()
                    assert_same(gpu.download(out), want, strict=True, what=f"{name} after {skip} allocations")
                    gpu.free(out)
                    break
                assert rc == gpu.CR_ERR_ALLOC, (name, skip, rc, lib.cr_last_error())
                assert b"out-of-memory" in lib.cr_last_error(), lib.cr_last_error()
                assert out.n_containers == 0 and not out.bitmap_data and not out.keys and not out._alloc_base, \
                    (name, skip, "output not reset")
                failures += 1
            else:
                pytest.fail(f"{name}: still failing after 16 allocations")
            assert failures >= 1, name
            # and the library is still usable: the same call again, with no injection
            rc, out = fn()
            assert rc == 0, (name, lib.cr_last_error())
            gpu.synchronize()
            assert_same(gpu.download(out), want, strict=True, what=f"{name} after the failures")
            gpu.free(out)
    finally:
        lib.cr_debug_fail_device_allocs(0, 0)
        for g in owned:
            gpu.free(g)
        del keep


def _same_batch(a, b):
    for k, v in vars(a).items():
        w = getattr(b, k)
        assert (np.array_equal(v, w) if isinstance(v, np.ndarray) else v == w), k


def test_batch_alloc_failure_returns_cr_err_alloc(gpu):
    """The batch API's producing calls under the same injected failures."""
    lib = gpu.load()
    rng = np.random.default_rng(41)
    lists = []
    for b in range(3):
        ids = np.unique(rng.integers(0, 1 << 22, 60000 * (b + 1), dtype=np.uint64)).astype(np.uint32)
        lists.append(orc.Lite.from_sorted_ids(ids).run_optimize().containers())
    arrays = [gpu._container_array(c) for c in lists]
    ptrs = (C.c_void_p * 3)(*[C.addressof(a[0]) for a in arrays])
    counts = (C.c_uint32 * 3)(*[len(c) for c in lists])
    idx = np.array([0, 2], dtype=np.uint32)
    B = gpu.upload_batch(lists)
    P = gpu.promote_batch(B)

    def run(f):
        out = gpu.RoaringBatch()
        return f(out), out
    calls = [
        ("upload_batch", lambda: run(lambda o: lib.cr_upload_batch(ptrs, counts, 3, None, C.byref(o)))),
        ("promote_batch", lambda: run(lambda o: lib.cr_promote_batch(C.byref(B), None, C.byref(o)))),
        ("batch_multi_and", lambda: run(lambda o: lib.cr_batch_multi_and(C.byref(P), idx.ctypes.data, 2, None,
                                                                          C.byref(o)))),
    ]
    try:
        for name, fn in calls:
            _say("batch alloc failure", name)
            rc, ref = fn()
            assert rc == 0, (name, lib.cr_last_error())
            gpu.synchronize()
            want = gpu.download_batch(ref)
            gpu.free_batch(ref)
            failures = 0
            for skip in range(16):
                lib.cr_debug_fail_device_allocs(skip, 1)
                rc, out = fn()
                lib.cr_debug_fail_device_allocs(0, 0)
                if rc == 0:
                    gpu.synchronize()
                    _same_batch(gpu.download_batch(out), want)
                    gpu.free_batch(out)
                    break
                assert rc == gpu.CR_ERR_ALLOC, (name, skip, rc, lib.cr_last_error())
                assert out.total_containers == 0 and not out._alloc_base, (name, skip, "output not reset")
                failures += 1
            else:
                pytest.fail(f"{name}: still failing after 16 allocations")
            assert failures >= 1, name
    finally:
        lib.cr_debug_fail_device_allocs(0, 0)
        gpu.free_batch(P)
        gpu.free_batch(B)
        del arrays

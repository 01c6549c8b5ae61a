"""GPU bitmaps of every shape the conversion and serialization tests use:
(GpuRoaring, its stored ids as a sorted numpy array, or None when the test
does not know them)."""
import zlib

import numpy as np

import orc


def run_heavy_ids(rng, U):
    """Random runs of mixed lengths, one full key, odd word boundaries."""
    parts = []
    for key in range(U // 65536):
        base = key * 65536
        kind = key % 4
        if kind == 0:
            parts.append(base + np.arange(65536))  # full container -> one run [0, 65535]
        elif kind == 1:
            starts = np.sort(rng.choice(65536 // 64, 300, replace=False)) * 64
            for s in starts:
                parts.append(base + np.arange(s + int(rng.integers(0, 5)), s + int(rng.integers(5, 64))))
        elif kind == 2:
            parts.append(base + np.arange(31, 40000))  # head and tail words partial
        else:
            parts.append(base + np.unique(rng.integers(0, 65536, 900)))
    return np.unique(np.concatenate(parts)).astype(np.uint32)


def make_bitmap(gpu, kind):
    """(GpuRoaring, stored ids as a sorted numpy array or None when not known)."""
    rng = np.random.default_rng(zlib.crc32(kind.encode()))
    if kind == "ids_keep":
        ids = rng.integers(0, 1 << 22, 200000, dtype=np.uint64).astype(np.uint32)
        return gpu.upload_from_ids(ids, 1 << 22, orc.PROMOTE_KEEP_DEFAULT), np.unique(ids)
    if kind == "ids_all_bitmap":
        ids = rng.integers(0, 1 << 21, 5000, dtype=np.uint64).astype(np.uint32)
        return gpu.upload_from_ids(ids, 1 << 21, orc.PROMOTE_ALL), np.unique(ids)
    if kind == "runs_mixed":
        U = 8 * 65536
        ids = run_heavy_ids(rng, U)
        lite = orc.Lite.from_sorted_ids(ids).run_optimize()
        g = gpu.upload_containers(lite.containers(), U, False, lite.cardinality(), orc.PROMOTE_KEEP_DEFAULT)
        assert g.n_run_containers > 0 and g.n_array_containers > 0
        return g, ids
    if kind == "arrays_only":
        U = 40 * 65536 + 5
        ids = np.unique(rng.integers(0, U, 12000, dtype=np.uint64)).astype(np.uint32)
        lite = orc.Lite.from_sorted_ids(ids)
        g = gpu.upload_containers(lite.containers(), U, False, lite.cardinality(), orc.PROMOTE_KEEP_DEFAULT)
        assert g.n_array_containers == g.n_containers > 0 and g.key_index
        return g, ids
    if kind == "negated_odd_u":
        U = 100003
        keep = rng.random(U) < 0.9
        ids = np.nonzero(keep)[0].astype(np.uint32)
        g = gpu.upload_from_ids(ids, U, orc.PROMOTE_KEEP_DEFAULT)
        assert g.negated
        return g, np.nonzero(~keep)[0].astype(np.uint32)
    if kind == "negated_runs":
        U = 5 * 65536 + 77
        ids = np.concatenate([np.arange(0, 200000), np.arange(200100, U)]).astype(np.uint32)
        g = gpu.upload_from_ids(ids, U, orc.PROMOTE_KEEP_DEFAULT)
        assert g.negated
        return g, np.arange(200000, 200100, dtype=np.uint32)
    if kind == "empty":
        return gpu.upload_from_ids(np.zeros(0, np.uint32), 1000, orc.PROMOTE_KEEP_DEFAULT), np.zeros(0, np.uint32)
    if kind == "negated_empty":
        g = gpu.upload_from_ids(np.arange(1000, dtype=np.uint32), 1000, orc.PROMOTE_KEEP_DEFAULT)
        assert g.negated and g.n_containers == 0
        return g, np.zeros(0, np.uint32)
    if kind == "setop_result":
        a = gpu.upload_from_ids(np.arange(0, 150000, dtype=np.uint32), 1 << 20, orc.PROMOTE_KEEP_DEFAULT)
        b = gpu.upload_from_ids(np.arange(70000, 300000, 3, dtype=np.uint32), 1 << 20, orc.PROMOTE_KEEP_DEFAULT)
        g = gpu.set_operation(a, b, orc.AND)
        gpu.free(a)
        gpu.free(b)
        return g, None
    raise ValueError(kind)


KINDS = ["ids_keep", "ids_all_bitmap", "runs_mixed", "arrays_only", "negated_odd_u", "negated_runs", "empty", "negated_empty",
         "setop_result"]

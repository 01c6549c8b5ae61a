"""ctypes binding of libcuroaring_amd.so (the C-ABI in include/cu_roaring_abi.h).

Used by the tests and bench.py.  Every call goes through the C-ABI into the HIP
library; there is no CPU fallback: load() raises when the built library is
missing.  Device buffers come from torch (plumbing only).
"""
from __future__ import annotations

import ctypes as C
import os
from types import SimpleNamespace
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.dirname(_HERE)
LIB_PATH = os.path.join(PKG_DIR, "lib", "libcuroaring_amd.so")

CR_OK = 0
CR_ERR_HIP, CR_ERR_INVALID, CR_ERR_ALLOC, CR_ERR_UNSUPPORTED, CR_ERR_RANGE = 1, 2, 3, 4, 5
ARRAY, BITMAP, RUN = 0, 1, 2
AND, OR, ANDNOT, XOR = 0, 1, 2, 3
PROMOTE_KEEP_DEFAULT = 4096
PROMOTE_ALL = 0
PROMOTE_AUTO = 0xFFFFFFFF
TC_BITSET, TC_ARRAY, TC_RUN = 1, 2, 3
QUERY_CONTAINS, QUERY_WAVEFRONT, QUERY_WAVEFRONT_API, QUERY_CONTAINS_API, QUERY_PARTITIONED = 0, 1, 2, 3, 4

EXPORTS = [
    "cr_last_error", "cr_upload_from_ids", "cr_upload_from_device_ids", "cr_upload_from_bitset",
    "cr_upload_from_device_bitset", "cr_upload_containers", "cr_get_meta", "cr_set_operation", "cr_multi_and",
    "cr_free", "cr_free_async", "cr_resolve_auto_threshold", "cr_make_view", "cr_contains_batch",
    "cr_topk_filtered", "cr_topk_set_small_limit", "cr_device_l2_bytes", "cr_device_malloc", "cr_device_free", "cr_memcpy_h2d",
    "cr_memcpy_d2h", "cr_stream_synchronize", "cr_timing_enable", "cr_timing_report", "cr_mempool_trim",
    "cr_decompress_to_bitset", "cr_decompress_to_bitset_alloc", "cr_enumerate_ids", "cr_enumerate_ids_alloc",
    "cr_enumerate_ids_noalloc", "cr_cardinality",
    "cr_promote_to_bitmap", "cr_promote_auto", "cr_deep_copy",
    "cr_portable_size_in_bytes", "cr_portable_serialize", "cr_portable_deserialize",
    "cr_upload_batch", "cr_free_batch", "cr_promote_batch", "cr_batch_make_view", "cr_batch_multi_and",
    "cr_batch_decompress", "cr_batch_contains", "cr_batch_view_contains", "cr_debug_fail_device_allocs",
]


class GpuRoaring(C.Structure):
    """cr_gpu_roaring == cu_roaring::GpuRoaring (include/cu_roaring/types.cuh:15-54)."""
    _fields_ = [
        ("keys", C.c_void_p),
        ("types", C.c_void_p),
        ("offsets", C.c_void_p),
        ("cardinalities", C.c_void_p),
        ("n_containers", C.c_uint32),
        ("universe_size", C.c_uint32),
        ("total_cardinality", C.c_uint64),
        ("bitmap_data", C.c_void_p),
        ("n_bitmap_containers", C.c_uint32),
        ("array_data", C.c_void_p),
        ("n_array_containers", C.c_uint32),
        ("array_pool_bytes", C.c_uint32),
        ("run_data", C.c_void_p),
        ("n_run_containers", C.c_uint32),
        ("run_pool_bytes", C.c_uint32),
        ("key_index", C.c_void_p),
        ("max_key", C.c_uint32),
        ("negated", C.c_bool),
        ("_alloc_base", C.c_void_p),
    ]


class GpuRoaringView(C.Structure):
    _fields_ = [
        ("keys", C.c_void_p),
        ("types", C.c_void_p),
        ("offsets", C.c_void_p),
        ("cardinalities", C.c_void_p),
        ("n_containers", C.c_uint32),
        ("bitmap_data", C.c_void_p),
        ("array_data", C.c_void_p),
        ("run_data", C.c_void_p),
        ("key_index", C.c_void_p),
        ("max_key", C.c_uint32),
        ("all_bitmap", C.c_bool),
        ("negated", C.c_bool),
    ]


class RoaringBatch(C.Structure):
    """cr_roaring_batch == cu_roaring::v2::GpuRoaringBatch (v2/include/cu_roaring_v2/types.cuh:37-86)."""
    _fields_ = [
        ("n_bitmaps", C.c_uint32), ("total_containers", C.c_uint32), ("n_bitmap_containers_total", C.c_uint32),
        ("array_pool_bytes", C.c_uint32), ("run_pool_bytes", C.c_uint32),
        ("container_starts", C.c_void_p), ("key_index_starts", C.c_void_p),
        ("keys", C.c_void_p), ("types", C.c_void_p), ("offsets", C.c_void_p), ("cardinalities", C.c_void_p),
        ("key_indices", C.c_void_p), ("bitmap_data", C.c_void_p), ("array_data", C.c_void_p),
        ("run_data", C.c_void_p),
        ("host_total_cardinalities", C.POINTER(C.c_uint64)), ("host_universe_sizes", C.POINTER(C.c_uint32)),
        ("host_container_starts", C.POINTER(C.c_uint32)), ("host_key_index_starts", C.POINTER(C.c_uint32)),
        ("host_n_bitmap_containers", C.POINTER(C.c_uint32)),
        ("_alloc_base", C.c_void_p), ("_host_meta_base", C.c_void_p),
    ]


class BatchView(C.Structure):
    """cr_batch_view == cu_roaring::v2::GpuRoaringView (v2/include/cu_roaring_v2/types.cuh:95-107)."""
    _fields_ = [
        ("n_containers", C.c_uint32), ("max_key", C.c_uint32),
        ("keys", C.c_void_p), ("types", C.c_void_p), ("offsets", C.c_void_p), ("cardinalities", C.c_void_p),
        ("key_index", C.c_void_p), ("bitmap_data", C.c_void_p), ("array_data", C.c_void_p), ("run_data", C.c_void_p),
    ]


class HostContainer(C.Structure):
    _fields_ = [("key", C.c_uint16), ("typecode", C.c_uint8), ("cardinality", C.c_int32), ("data", C.c_void_p)]


class Meta(C.Structure):
    _fields_ = [("n_containers", C.c_uint32), ("n_bitmap_containers", C.c_uint32),
                ("n_array_containers", C.c_uint32), ("n_run_containers", C.c_uint32),
                ("universe_size", C.c_uint32), ("total_bytes", C.c_size_t)]


assert C.sizeof(GpuRoaring) == 120 and C.sizeof(GpuRoaringView) == 80

_lib = None


class CrError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def load(path: Optional[str] = None):
    """Load the HIP library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise RuntimeError(f"libcuroaring_amd.so not built at {p}: run `make -C cu-roaring-bitmap_amd` "
                           f"(or __graft_entry__.build())")
    L = C.CDLL(p)
    P = C.POINTER
    L.cr_last_error.restype = C.c_char_p
    sigs = {
        "cr_upload_from_ids": [C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p, C.c_uint32, P(GpuRoaring)],
        "cr_upload_from_device_ids": [C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p, C.c_uint32, P(GpuRoaring)],
        "cr_upload_from_bitset": [C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p, P(GpuRoaring)],
        "cr_upload_from_device_bitset": [C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p, P(GpuRoaring)],
        "cr_upload_containers": [C.c_void_p, C.c_uint32, C.c_uint32, C.c_bool, C.c_uint64, C.c_void_p, C.c_uint32,
                                 P(GpuRoaring)],
        "cr_get_meta": [C.c_void_p, C.c_uint32, P(Meta)],
        "cr_set_operation": [P(GpuRoaring), P(GpuRoaring), C.c_uint32, C.c_void_p, P(GpuRoaring)],
        "cr_multi_and": [C.c_void_p, C.c_uint32, C.c_void_p, P(GpuRoaring)],
        "cr_free": [P(GpuRoaring)],
        "cr_free_async": [P(GpuRoaring), C.c_void_p],
        "cr_resolve_auto_threshold": [C.c_uint32, C.c_int, P(C.c_uint32)],
        "cr_make_view": [P(GpuRoaring), P(GpuRoaringView)],
        "cr_contains_batch": [P(GpuRoaringView), C.c_void_p, C.c_uint64, C.c_void_p, C.c_uint32, C.c_void_p],
        "cr_topk_set_small_limit": [C.c_uint32],
        "cr_topk_filtered": [C.c_void_p, C.c_uint64, C.c_void_p, C.c_uint32, C.c_uint32, P(GpuRoaring), C.c_uint32,
                             C.c_void_p, C.c_void_p, C.c_void_p],
        "cr_device_l2_bytes": [C.c_int, P(C.c_uint64)],
        "cr_device_malloc": [P(C.c_void_p), C.c_size_t],
        "cr_device_free": [C.c_void_p],
        "cr_memcpy_h2d": [C.c_void_p, C.c_void_p, C.c_size_t],
        "cr_memcpy_d2h": [C.c_void_p, C.c_void_p, C.c_size_t],
        "cr_stream_synchronize": [C.c_void_p],
        "cr_timing_enable": [C.c_int],
        "cr_mempool_trim": [C.c_int, C.c_size_t],
        "cr_timing_report": [C.c_char_p, C.c_size_t],
        "cr_decompress_to_bitset": [P(GpuRoaring), C.c_void_p, C.c_uint32, C.c_void_p],
        "cr_decompress_to_bitset_alloc": [P(GpuRoaring), C.c_void_p, P(C.c_void_p), P(C.c_uint32)],
        "cr_enumerate_ids": [P(GpuRoaring), C.c_void_p, C.c_uint64, C.c_void_p],
        "cr_enumerate_ids_alloc": [P(GpuRoaring), C.c_void_p, P(C.c_void_p), P(C.c_uint64)],
        "cr_enumerate_ids_noalloc": [P(GpuRoaring), C.c_void_p, C.c_uint64, C.c_void_p],
        "cr_cardinality": [P(GpuRoaring), C.c_void_p, P(C.c_uint64)],
        "cr_promote_to_bitmap": [P(GpuRoaring), C.c_void_p, P(GpuRoaring)],
        "cr_promote_auto": [P(GpuRoaring), C.c_void_p, C.c_int, P(GpuRoaring)],
        "cr_deep_copy": [P(GpuRoaring), C.c_void_p, P(GpuRoaring)],
        "cr_portable_size_in_bytes": [P(GpuRoaring), C.c_void_p, P(C.c_size_t)],
        "cr_portable_serialize": [P(GpuRoaring), C.c_void_p, C.c_void_p, C.c_size_t, P(C.c_size_t)],
        "cr_portable_deserialize": [C.c_void_p, C.c_size_t, C.c_uint32, C.c_void_p, C.c_uint32, P(GpuRoaring)],
        "cr_upload_batch": [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, P(RoaringBatch)],
        "cr_free_batch": [P(RoaringBatch)],
        "cr_promote_batch": [P(RoaringBatch), C.c_void_p, P(RoaringBatch)],
        "cr_batch_make_view": [P(RoaringBatch), C.c_uint32, P(BatchView)],
        "cr_batch_multi_and": [P(RoaringBatch), C.c_void_p, C.c_uint32, C.c_void_p, P(RoaringBatch)],
        "cr_batch_decompress": [P(RoaringBatch), C.c_void_p, C.c_uint64, C.c_void_p],
        "cr_batch_contains": [P(RoaringBatch), C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p],
        "cr_batch_view_contains": [P(BatchView), C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p],
        "cr_debug_fail_device_allocs": [C.c_uint32, C.c_uint32],
    }
    for name, args in sigs.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = C.c_int
    L.cr_topk_set_small_limit.restype = C.c_uint32
    _lib = L
    return L


def _check(rc: int, what: str):
    if rc != CR_OK:
        raise CrError(rc, f"{what}: {_lib.cr_last_error().decode(errors='replace')}")


def _stream(stream) -> Optional[int]:
    if stream is None:
        return None
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream  # torch.cuda.Stream


def _dptr(t) -> int:
    return t.data_ptr()


# ---- uploads ---------------------------------------------------------------
def upload_from_ids(ids, universe: int, threshold: int = PROMOTE_AUTO, stream=None) -> GpuRoaring:
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    out = GpuRoaring()
    _check(load().cr_upload_from_ids(ids.ctypes.data if ids.size else None, ids.size, universe, _stream(stream),
                                     threshold, C.byref(out)), "upload_from_ids")
    return out


def upload_from_device_ids(d_ids, universe: int, threshold: int = PROMOTE_AUTO, stream=None) -> GpuRoaring:
    """d_ids: a torch int32/uint32 CUDA tensor (read as uint32)."""
    out = GpuRoaring()
    n = d_ids.numel()
    _check(load().cr_upload_from_device_ids(_dptr(d_ids) if n else None, n, universe, _stream(stream), threshold,
                                            C.byref(out)), "upload_from_device_ids")
    return out


def upload_from_bitset(words, universe: int, stream=None) -> GpuRoaring:
    words = np.ascontiguousarray(words, dtype=np.uint32)
    out = GpuRoaring()
    _check(load().cr_upload_from_bitset(words.ctypes.data if words.size else None, words.size, universe,
                                        _stream(stream), C.byref(out)), "upload_from_bitset")
    return out


def upload_from_device_bitset(d_words, universe: int, stream=None) -> GpuRoaring:
    out = GpuRoaring()
    n = d_words.numel()
    _check(load().cr_upload_from_device_bitset(_dptr(d_words) if n else None, n, universe, _stream(stream),
                                               C.byref(out)), "upload_from_device_bitset")
    return out


def _container_array(containers):
    arr = (HostContainer * max(1, len(containers)))()
    keep = []
    for i, (key, tc, card, payload) in enumerate(containers):
        p = np.ascontiguousarray(payload)
        keep.append(p)
        arr[i] = HostContainer(key, tc, card, p.ctypes.data if p.size else None)
    return arr, keep


def upload_containers(containers, universe: int = 0, complemented: bool = False, logical_cardinality: int = 0,
                      threshold: int = PROMOTE_AUTO, stream=None) -> GpuRoaring:
    """containers: [(key, typecode, cardinality|n_runs, payload ndarray)] sorted by key."""
    arr, keep = _container_array(containers)
    out = GpuRoaring()
    _check(load().cr_upload_containers(arr, len(containers), universe, complemented, logical_cardinality,
                                       _stream(stream), threshold, C.byref(out)), "upload_containers")
    del keep
    return out


def get_meta(containers) -> Meta:
    arr, keep = _container_array(containers)
    m = Meta()
    _check(load().cr_get_meta(arr, len(containers), C.byref(m)), "get_meta")
    return m


# ---- set operations ----------------------------------------------------------
def set_operation(a: GpuRoaring, b: GpuRoaring, op: int, stream=None) -> GpuRoaring:
    out = GpuRoaring()
    _check(load().cr_set_operation(C.byref(a), C.byref(b), op, _stream(stream), C.byref(out)), "set_operation")
    return out


def multi_and(bitmaps: Sequence[GpuRoaring], stream=None) -> GpuRoaring:
    arr = (GpuRoaring * max(1, len(bitmaps)))()
    for i, b in enumerate(bitmaps):
        arr[i] = b
    out = GpuRoaring()
    _check(load().cr_multi_and(arr, len(bitmaps), _stream(stream), C.byref(out)), "multi_and")
    return out


def free(g: GpuRoaring):
    _check(load().cr_free(C.byref(g)), "free")


def free_async(g: GpuRoaring, stream=None):
    _check(load().cr_free_async(C.byref(g), _stream(stream)), "free_async")


def resolve_auto_threshold(universe: int, device: int = -1) -> int:
    t = C.c_uint32()
    _check(load().cr_resolve_auto_threshold(universe, device, C.byref(t)), "resolve_auto_threshold")
    return t.value


def device_l2_bytes(device: int = -1) -> int:
    v = C.c_uint64()
    _check(load().cr_device_l2_bytes(device, C.byref(v)), "device_l2_bytes")
    return v.value


def make_view(g: GpuRoaring) -> GpuRoaringView:
    v = GpuRoaringView()
    _check(load().cr_make_view(C.byref(g), C.byref(v)), "make_view")
    return v


def contains_batch(g: GpuRoaring, d_ids, d_out, mode: int = QUERY_CONTAINS, stream=None):
    """d_ids / d_out: CUDA tensors of n uint32 (int32 storage); asynchronous."""
    v = make_view(g)
    n = d_ids.numel()
    _check(load().cr_contains_batch(C.byref(v), _dptr(d_ids), n, _dptr(d_out), mode, _stream(stream)),
           "contains_batch")


def topk_set_small_limit(rows: int) -> int:
    """Rows at or below which the top-k keeps every estimate and selects per
    query (capped at 262144; 0 turns that path off).  Returns the previous limit."""
    return int(load().cr_topk_set_small_limit(rows))


def topk_filtered(d_base, d_queries, k: int, filt: Optional[GpuRoaring], d_dist, d_ids, stream=None):
    n_base, dim = d_base.shape
    nq = d_queries.shape[0]
    _check(load().cr_topk_filtered(_dptr(d_base), n_base, _dptr(d_queries), nq, dim,
                                   C.byref(filt) if filt is not None else None, k, _dptr(d_dist), _dptr(d_ids),
                                   _stream(stream)), "topk_filtered")


# ---- conversions (stream-ordered, no synchronisation) -------------------------
NO_BOUND = 0xFFFFFFFFFFFFFFFF


def decompress_to_bitset(g: GpuRoaring, d_out, n_words: Optional[int] = None, stream=None):
    """decompress_to_bitset into d_out (a CUDA tensor of >= n_words 32-bit words)."""
    if n_words is None:
        n_words = d_out.numel()
    _check(load().cr_decompress_to_bitset(C.byref(g), _dptr(d_out), n_words, _stream(stream)),
           "decompress_to_bitset")


def decompress_to_bitset_alloc(g: GpuRoaring, stream=None):
    """The allocating overload: (device pointer or None, n_words); free with device_free."""
    p, n = C.c_void_p(), C.c_uint32()
    _check(load().cr_decompress_to_bitset_alloc(C.byref(g), _stream(stream), C.byref(p), C.byref(n)),
           "decompress_to_bitset_alloc")
    return p.value, n.value


def enumerate_ids(g: GpuRoaring, d_out, capacity: int = NO_BOUND, stream=None):
    """enumerate_ids into d_out (a CUDA int64 tensor)."""
    _check(load().cr_enumerate_ids(C.byref(g), _dptr(d_out), capacity, _stream(stream)), "enumerate_ids")


def cardinality(g: GpuRoaring, stream=None) -> int:
    """The logical cardinality counted on the device (set-operation results included)."""
    n = C.c_uint64()
    _check(load().cr_cardinality(C.byref(g), _stream(stream), C.byref(n)), "cardinality")
    return n.value


def enumerate_ids_noalloc(g: GpuRoaring, d_out, capacity: int = NO_BOUND, stream=None):
    """enumerate_ids into d_out with no device allocation (the library's fixed per-device scratch)."""
    _check(load().cr_enumerate_ids_noalloc(C.byref(g), _dptr(d_out), capacity, _stream(stream)),
           "enumerate_ids_noalloc")


def enumerate_ids_alloc(g: GpuRoaring, stream=None):
    """The allocating overload: (device pointer or None, n_ids); free with device_free."""
    p, n = C.c_void_p(), C.c_uint64()
    _check(load().cr_enumerate_ids_alloc(C.byref(g), _stream(stream), C.byref(p), C.byref(n)), "enumerate_ids_alloc")
    return p.value, n.value


def promote_to_bitmap(g: GpuRoaring, stream=None) -> GpuRoaring:
    out = GpuRoaring()
    _check(load().cr_promote_to_bitmap(C.byref(g), _stream(stream), C.byref(out)), "promote_to_bitmap")
    return out


def promote_auto(g: GpuRoaring, stream=None, device: int = -1) -> GpuRoaring:
    out = GpuRoaring()
    _check(load().cr_promote_auto(C.byref(g), _stream(stream), device, C.byref(out)), "promote_auto")
    return out


def deep_copy(g: GpuRoaring, stream=None) -> GpuRoaring:
    out = GpuRoaring()
    _check(load().cr_deep_copy(C.byref(g), _stream(stream), C.byref(out)), "deep_copy")
    return out


# ---- Roaring portable format ------------------------------------------------------
def portable_size_in_bytes(g: GpuRoaring, stream=None) -> int:
    n = C.c_size_t()
    _check(load().cr_portable_size_in_bytes(C.byref(g), _stream(stream), C.byref(n)), "portable_size_in_bytes")
    return n.value


def portable_serialize(g: GpuRoaring, stream=None) -> bytes:
    """The logical set of g in the Roaring portable format."""
    n = portable_size_in_bytes(g, stream)
    buf = C.create_string_buffer(max(n, 1))
    w = C.c_size_t()
    _check(load().cr_portable_serialize(C.byref(g), _stream(stream), buf, n, C.byref(w)), "portable_serialize")
    return buf.raw[:w.value]


def portable_deserialize(data: bytes, universe: int = 0, threshold: int = PROMOTE_AUTO, stream=None) -> GpuRoaring:
    """upload() of a portable-format bitmap (universe 0: upload(bm); else upload(bm, U))."""
    out = GpuRoaring()
    buf = C.create_string_buffer(bytes(data), max(len(data), 1))
    _check(load().cr_portable_deserialize(buf, len(data), universe, _stream(stream), threshold, C.byref(out)),
           "portable_deserialize")
    return out


# ---- the batch API (the reference's v2) -------------------------------------------
def upload_batch(bitmaps, stream=None) -> RoaringBatch:
    """bitmaps: a list of container lists, each [(key, typecode, card, ndarray)]."""
    arrays = [_container_array(c) for c in bitmaps]
    ptrs = (C.c_void_p * max(1, len(bitmaps)))(*[C.addressof(a[0]) if len(a[0]) else None for a in arrays])
    counts = (C.c_uint32 * max(1, len(bitmaps)))(*[len(c) for c in bitmaps])
    out = RoaringBatch()
    _check(load().cr_upload_batch(ptrs, counts, len(bitmaps), _stream(stream), C.byref(out)), "upload_batch")
    return out


def free_batch(b: RoaringBatch):
    _check(load().cr_free_batch(C.byref(b)), "free_batch")


def promote_batch(b: RoaringBatch, stream=None) -> RoaringBatch:
    out = RoaringBatch()
    _check(load().cr_promote_batch(C.byref(b), _stream(stream), C.byref(out)), "promote_batch")
    return out


def batch_make_view(b: RoaringBatch, idx: int) -> BatchView:
    v = BatchView()
    _check(load().cr_batch_make_view(C.byref(b), idx, C.byref(v)), "make_view")
    return v


def batch_multi_and(b: RoaringBatch, indices, stream=None) -> RoaringBatch:
    idx = np.ascontiguousarray(indices, dtype=np.uint32)
    out = RoaringBatch()
    _check(load().cr_batch_multi_and(C.byref(b), idx.ctypes.data if idx.size else None, idx.size, _stream(stream),
                                     C.byref(out)), "multi_and")
    return out


def batch_decompress(b: RoaringBatch, d_bitsets, words_each: int, stream=None):
    _check(load().cr_batch_decompress(C.byref(b), _dptr(d_bitsets), words_each, _stream(stream)), "decompress_batch")


def batch_contains(b: RoaringBatch, d_ids, d_out, bitmap: int = 0, d_bitmap_idx=None, stream=None):
    """d_out[i] = bitmap (d_bitmap_idx[i] or `bitmap`) holds d_ids[i]; d_out is a uint8 CUDA tensor."""
    _check(load().cr_batch_contains(C.byref(b), _dptr(d_bitmap_idx) if d_bitmap_idx is not None else None, bitmap,
                                    _dptr(d_ids), d_ids.numel(), _dptr(d_out), _stream(stream)), "batch_contains")


def batch_view_contains(v: BatchView, d_ids, d_out, stream=None):
    _check(load().cr_batch_view_contains(C.byref(v), _dptr(d_ids), d_ids.numel(), _dptr(d_out), _stream(stream)),
           "batch_view_contains")


def download_batch(b: RoaringBatch) -> SimpleNamespace:
    """Host copy of a batch (same fields as the oracle's HostBatch); the
    metadata arrays hold the batch's live slices only."""
    n, T = b.n_bitmaps, b.total_containers
    h = lambda p, k: np.ctypeslib.as_array(p, shape=(k,)).copy() if (k and p) else np.zeros(0)
    hcs = h(b.host_container_starts, n + 1).astype(np.uint32) if n else np.zeros(0, np.uint32)
    hks = h(b.host_key_index_starts, n + 1).astype(np.uint32) if n else np.zeros(0, np.uint32)
    kidx = int(hks[-1]) if n else 0
    return SimpleNamespace(
        n_bitmaps=n, total_containers=T, n_bitmap_containers_total=b.n_bitmap_containers_total,
        array_pool_bytes=b.array_pool_bytes, run_pool_bytes=b.run_pool_bytes,
        container_starts=_d2h(b.container_starts, n + 1 if n else 0, np.uint32),
        key_index_starts=_d2h(b.key_index_starts, n + 1 if n else 0, np.uint32),
        keys=_d2h(b.keys, T, np.uint16), types=_d2h(b.types, T, np.uint8), offsets=_d2h(b.offsets, T, np.uint32),
        cards=_d2h(b.cardinalities, T, np.uint16), key_indices=_d2h(b.key_indices, kidx, np.uint16),
        bitmap_data=_d2h(b.bitmap_data, b.n_bitmap_containers_total * 1024, np.uint64),
        array_data=_d2h(b.array_data, b.array_pool_bytes // 2, np.uint16),
        run_data=_d2h(b.run_data, b.run_pool_bytes // 2, np.uint16),
        host_total_cardinalities=h(b.host_total_cardinalities, n).astype(np.uint64) if n else np.zeros(0, np.uint64),
        host_universe_sizes=h(b.host_universe_sizes, n).astype(np.uint32) if n else np.zeros(0, np.uint32),
        host_container_starts=hcs, host_key_index_starts=hks,
        host_n_bitmap_containers=h(b.host_n_bitmap_containers, n).astype(np.uint32) if n else np.zeros(0, np.uint32),
    )


def device_free(ptr):
    if ptr:
        _check(load().cr_device_free(ptr), "device_free")


def synchronize(stream=None):
    _check(load().cr_stream_synchronize(_stream(stream)), "stream_synchronize")


def timing_enable(on: bool = True, every: int = 1):
    """Start (or stop) per-kernel HIP-event timing inside the library; clears records.
    every > 1 times only every every-th launch of each kernel."""
    _check(load().cr_timing_enable(max(1, int(every)) if on else 0), "timing_enable")


def timing_report() -> dict:
    """{kernel_name: (launches, total_ms, median_ms)} for the launches since timing_enable()."""
    buf = C.create_string_buffer(1 << 16)
    _check(load().cr_timing_report(buf, len(buf)), "timing_report")
    out = {}
    for line in buf.value.decode().splitlines():
        name, n, ms, med = line.split()
        out[name] = (int(n), float(ms), float(med))
    return out


# ---- download to host (canonical comparison) -----------------------------------
def _d2h(ptr, n, dtype):
    a = np.zeros(n, dtype=dtype)
    if n and ptr:
        _check(load().cr_memcpy_d2h(a.ctypes.data, ptr, a.nbytes), "memcpy_d2h")
    return a


def download(g: GpuRoaring) -> SimpleNamespace:
    """Host copy of every field and pool (same shape as the oracle's HostRoaring)."""
    n = g.n_containers
    kidx = _d2h(g.key_index, g.max_key + 1, np.uint16) if g.key_index else None
    return SimpleNamespace(
        keys=_d2h(g.keys, n, np.uint16),
        types=_d2h(g.types, n, np.uint8),
        offsets=_d2h(g.offsets, n, np.uint32),
        cards=_d2h(g.cardinalities, n, np.uint16),
        n_containers=n,
        universe_size=g.universe_size,
        total_cardinality=g.total_cardinality,
        bitmap_data=_d2h(g.bitmap_data, g.n_bitmap_containers * 1024, np.uint64),
        n_bitmap_containers=g.n_bitmap_containers,
        array_data=_d2h(g.array_data, g.array_pool_bytes // 2, np.uint16),
        n_array_containers=g.n_array_containers,
        array_pool_bytes=g.array_pool_bytes,
        run_data=_d2h(g.run_data, g.run_pool_bytes // 2, np.uint16),
        n_run_containers=g.n_run_containers,
        run_pool_bytes=g.run_pool_bytes,
        key_index=kidx,
        max_key=g.max_key,
        negated=bool(g.negated),
    )

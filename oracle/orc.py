"""ctypes wrapper of the CPU oracle (oracle/lib/liborc.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() (as the
checker) and bench.py's cpu_baseline leg.  The product library never loads it.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "lib", "liborc.so")
# The same sources built for x86-64-v4 (AVX-512): the CPU baselines run from it
# when the host supports that level, so a baseline is never held to AVX2 on an
# AVX-512 machine.  The checker functions always come from the v3 build.
_LIB_V4_PATH = os.path.join(_HERE, "lib", "liborc_x86_64_v4.so")
_V4_FLAGS = ("avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl")

ARRAY, BITMAP, RUN = 0, 1, 2
AND, OR, ANDNOT, XOR = 0, 1, 2, 3
PROMOTE_KEEP_DEFAULT = 4096
PROMOTE_ALL = 0
PROMOTE_AUTO = 0xFFFFFFFF
TC_BITSET, TC_ARRAY, TC_RUN = 1, 2, 3
DEFAULT_L2 = 4 * 1024 * 1024  # the reference's fallback L2 size (src/promote.cu:348-352)


class _OrcRoaring(C.Structure):
    _fields_ = [
        ("keys", C.POINTER(C.c_uint16)),
        ("types", C.POINTER(C.c_uint8)),
        ("offsets", C.POINTER(C.c_uint32)),
        ("cards", C.POINTER(C.c_uint16)),
        ("n_containers", C.c_uint32),
        ("universe_size", C.c_uint32),
        ("total_cardinality", C.c_uint64),
        ("bitmap_data", C.POINTER(C.c_uint64)),
        ("n_bitmap_containers", C.c_uint32),
        ("bitmap_pool_words", C.c_uint32),
        ("array_data", C.POINTER(C.c_uint16)),
        ("n_array_containers", C.c_uint32),
        ("array_pool_bytes", C.c_uint32),
        ("run_data", C.POINTER(C.c_uint16)),
        ("n_run_containers", C.c_uint32),
        ("run_pool_bytes", C.c_uint32),
        ("key_index", C.POINTER(C.c_uint16)),
        ("key_index_len", C.c_uint32),
        ("max_key", C.c_uint32),
        ("negated", C.c_int32),
    ]


class _OrcContainer(C.Structure):
    _fields_ = [
        ("key", C.c_uint16),
        ("typecode", C.c_uint8),
        ("card", C.c_int32),
        ("data", C.c_void_p),
    ]


_lib = None
_cpu_lib = None


def lib():
    """The checker; ORC_LIB_PATH, when set, names another build of it (the
    sanitizer build, tests/test_sanitizers.py)."""
    global _lib
    if _lib is None:
        _lib = _load(os.environ.get("ORC_LIB_PATH") or _LIB_PATH)
    return _lib


def host_supports_v4() -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    fl = set(line.split(":", 1)[1].split())
                    return all(x in fl for x in _V4_FLAGS)
    except OSError:
        pass
    return False


def cpu_lib():
    """The oracle build the CPU baselines run from: x86-64-v4 when the host has
    AVX-512 (and that build exists), else the x86-64-v3 one."""
    global _cpu_lib
    if _cpu_lib is None:
        use_v4 = not os.environ.get("ORC_LIB_PATH") and host_supports_v4() and os.path.exists(_LIB_V4_PATH)
        _cpu_lib = _load(_LIB_V4_PATH) if use_v4 else lib()
    return _cpu_lib


def cpu_isa() -> str:
    return "x86-64-v4" if cpu_lib() is not lib() else "x86-64-v3"


def _load(path):
    if not os.path.exists(path):
        raise RuntimeError(f"oracle library not built: {path} (run `make -C oracle`)")
    L = C.CDLL(path)
    P = C.POINTER
    L.orc_free.argtypes = [P(_OrcRoaring)]
    L.orc_resolve_auto_threshold.argtypes = [C.c_uint32, C.c_uint64]
    L.orc_resolve_auto_threshold.restype = C.c_uint32
    L.orc_upload_from_ids.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint64, P(_OrcRoaring)]
    L.orc_upload_from_bitset.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, P(_OrcRoaring)]
    L.orc_upload_packed.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_int, C.c_uint64, C.c_uint32,
                                    C.c_uint64, P(_OrcRoaring)]
    L.orc_set_operation.argtypes = [P(_OrcRoaring), P(_OrcRoaring), C.c_int, P(_OrcRoaring)]
    L.orc_multi_and.argtypes = [C.c_void_p, C.c_uint32, P(_OrcRoaring)]
    L.orc_contains.argtypes = [P(_OrcRoaring), C.c_uint32]
    L.orc_contains_many.argtypes = [P(_OrcRoaring), C.c_void_p, C.c_uint64, C.c_void_p]
    L.orc_decompress.argtypes = [P(_OrcRoaring), C.c_void_p, C.c_uint32]
    L.orc_true_cardinality.argtypes = [P(_OrcRoaring)]
    L.orc_true_cardinality.restype = C.c_uint64
    L.orc_enumerate_ids.argtypes = [P(_OrcRoaring), C.c_void_p]
    L.orc_enumerate_ids.restype = C.c_uint64
    L.orc_promote_to_bitmap.argtypes = [P(_OrcRoaring), P(_OrcRoaring)]
    L.orc_promote_to_bitmap.restype = C.c_int
    L.orc_deep_copy.argtypes = [P(_OrcRoaring), P(_OrcRoaring)]
    L.orc_deep_copy.restype = C.c_int
    for name in ("orc_upload_from_ids", "orc_upload_from_bitset", "orc_upload_packed",
                 "orc_set_operation", "orc_multi_and", "orc_contains"):
        getattr(L, name).restype = C.c_int
    # roaring-lite
    L.rl_create.restype = C.c_void_p
    L.rl_destroy.argtypes = [C.c_void_p]
    L.rl_from_sorted_ids.argtypes = [C.c_void_p, C.c_uint64]
    L.rl_from_sorted_ids.restype = C.c_void_p
    L.rl_from_ids.argtypes = [C.c_void_p, C.c_uint64]
    L.rl_from_ids.restype = C.c_void_p
    L.rl_copy.argtypes = [C.c_void_p]
    L.rl_copy.restype = C.c_void_p
    L.rl_run_optimize.argtypes = [C.c_void_p]
    L.rl_op.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
    L.rl_op.restype = C.c_void_p
    L.rl_flip.argtypes = [C.c_void_p, C.c_uint64, C.c_uint64]
    L.rl_flip.restype = C.c_void_p
    L.rl_contains.argtypes = [C.c_void_p, C.c_uint32]
    L.rl_contains.restype = C.c_int
    L.rl_contains_many.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p]
    L.rl_cardinality.argtypes = [C.c_void_p]
    L.rl_cardinality.restype = C.c_uint64
    L.rl_to_ids.argtypes = [C.c_void_p, C.c_void_p]
    L.rl_to_ids.restype = C.c_uint64
    L.rl_n_containers.argtypes = [C.c_void_p]
    L.rl_n_containers.restype = C.c_uint32
    L.rl_to_containers.argtypes = [C.c_void_p, C.c_void_p]
    L.rl_count_types.argtypes = [C.c_void_p, P(C.c_uint32), P(C.c_uint32), P(C.c_uint32)]
    L.rl_portable_size.argtypes = [C.c_void_p]
    L.rl_portable_size.restype = C.c_uint64
    L.rl_portable_serialize.argtypes = [C.c_void_p, C.c_void_p]
    L.rl_portable_serialize.restype = C.c_uint64
    L.rl_portable_deserialize.argtypes = [C.c_void_p, C.c_uint64, P(C.c_uint64)]
    L.rl_portable_deserialize.restype = C.c_void_p
    # generators
    L.orc_mt_bernoulli_ids.argtypes = [C.c_uint32, C.c_double, C.c_uint32, C.c_void_p, P(C.c_uint64)]
    L.orc_mt_raw.argtypes = [C.c_uint32, C.c_void_p, C.c_uint64]
    L.orc_splitmix64.argtypes = [C.c_uint64]
    L.orc_splitmix64.restype = C.c_uint64
    L.orc_topk_bruteforce.argtypes = [C.c_void_p, C.c_uint64, C.c_void_p, C.c_uint32, C.c_uint32,
                                      C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p, C.c_int]
    L.rl_from_words.argtypes = [C.c_void_p, C.c_uint64]
    L.rl_from_words.restype = C.c_void_p
    L.rl_slice.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32]
    L.rl_slice.restype = C.c_void_p
    # CPU baselines (cpu_baseline.c)
    for name in ("orc_cpu_upload_ids", "orc_cpu_setop", "orc_cpu_multi_and", "orc_cpu_contains",
                 "orc_cpu_config0", "orc_cpu_topk_fp32"):
        getattr(L, name).restype = C.c_double
    L.orc_cpu_upload_ids.argtypes = [C.c_void_p, C.c_uint64, C.c_uint32, C.c_int, P(_OrcRoaring)]
    L.orc_cpu_setop.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32, C.c_int, C.c_int, P(C.c_uint64),
                                P(C.c_uint64)]
    L.orc_cpu_multi_and.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_int, P(C.c_uint64), P(C.c_uint64)]
    L.orc_cpu_contains.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p, C.c_int]
    L.orc_cpu_config0.argtypes = [C.c_void_p, C.c_uint64, C.c_void_p, C.c_uint64, C.c_void_p, C.c_uint64,
                                  C.c_void_p, C.c_void_p, P(C.c_uint64)]
    L.orc_cpu_topk_fp32.argtypes = [C.c_void_p, C.c_uint64, C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p,
                                    C.c_uint32, C.c_void_p, C.c_void_p, C.c_int]
    return L


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data if a is not None and a.size else 0


@dataclass
class HostRoaring:
    """Host mirror of a GpuRoaring (types.cuh:15-54) with numpy pools."""
    keys: np.ndarray
    types: np.ndarray
    offsets: np.ndarray
    cards: np.ndarray
    n_containers: int
    universe_size: int
    total_cardinality: int
    bitmap_data: np.ndarray
    n_bitmap_containers: int
    array_data: np.ndarray
    n_array_containers: int
    array_pool_bytes: int
    run_data: np.ndarray
    n_run_containers: int
    run_pool_bytes: int
    key_index: Optional[np.ndarray]
    max_key: int
    negated: bool
    _c: Optional[_OrcRoaring] = field(default=None, repr=False)
    _keep: list = field(default_factory=list, repr=False)

    # -- conversion to the C struct (for feeding the oracle) --------------
    def as_c(self) -> _OrcRoaring:
        if self._c is not None:
            return self._c
        arrs = {
            "keys": np.ascontiguousarray(self.keys, dtype=np.uint16),
            "types": np.ascontiguousarray(self.types, dtype=np.uint8),
            "offsets": np.ascontiguousarray(self.offsets, dtype=np.uint32),
            "cards": np.ascontiguousarray(self.cards, dtype=np.uint16),
            "bitmap_data": np.ascontiguousarray(self.bitmap_data, dtype=np.uint64),
            "array_data": np.ascontiguousarray(self.array_data, dtype=np.uint16),
            "run_data": np.ascontiguousarray(self.run_data, dtype=np.uint16),
        }
        c = _OrcRoaring()
        ctypes_of = {"keys": C.c_uint16, "types": C.c_uint8, "offsets": C.c_uint32, "cards": C.c_uint16,
                     "bitmap_data": C.c_uint64, "array_data": C.c_uint16, "run_data": C.c_uint16}
        for k, a in arrs.items():
            self._keep.append(a)
            if a.size:
                setattr(c, k, a.ctypes.data_as(C.POINTER(ctypes_of[k])))
        if self.key_index is not None:
            ki = np.ascontiguousarray(self.key_index, dtype=np.uint16)
            self._keep.append(ki)
            c.key_index = ki.ctypes.data_as(C.POINTER(C.c_uint16))
            c.key_index_len = ki.size
        c.n_containers = self.n_containers
        c.universe_size = self.universe_size
        c.total_cardinality = self.total_cardinality
        c.n_bitmap_containers = self.n_bitmap_containers
        c.bitmap_pool_words = arrs["bitmap_data"].size
        c.n_array_containers = self.n_array_containers
        c.array_pool_bytes = self.array_pool_bytes
        c.n_run_containers = self.n_run_containers
        c.run_pool_bytes = self.run_pool_bytes
        c.max_key = self.max_key
        c.negated = 1 if self.negated else 0
        self._c = c
        return c


def _arr(ptr, n, dtype):
    if not ptr or n == 0:
        return np.zeros(0, dtype=dtype)
    return np.ctypeslib.as_array(ptr, shape=(n,)).astype(dtype, copy=True)


def _from_c(c: _OrcRoaring) -> HostRoaring:
    n = c.n_containers
    r = HostRoaring(
        keys=_arr(c.keys, n, np.uint16),
        types=_arr(c.types, n, np.uint8),
        offsets=_arr(c.offsets, n, np.uint32),
        cards=_arr(c.cards, n, np.uint16),
        n_containers=n,
        universe_size=c.universe_size,
        total_cardinality=c.total_cardinality,
        bitmap_data=_arr(c.bitmap_data, c.bitmap_pool_words, np.uint64),
        n_bitmap_containers=c.n_bitmap_containers,
        array_data=_arr(c.array_data, c.array_pool_bytes // 2, np.uint16),
        n_array_containers=c.n_array_containers,
        array_pool_bytes=c.array_pool_bytes,
        run_data=_arr(c.run_data, c.run_pool_bytes // 2, np.uint16),
        n_run_containers=c.n_run_containers,
        run_pool_bytes=c.run_pool_bytes,
        key_index=_arr(c.key_index, c.key_index_len, np.uint16) if c.key_index else None,
        max_key=c.max_key,
        negated=bool(c.negated),
    )
    lib().orc_free(C.byref(c))
    return r


def as_host(r) -> HostRoaring:
    """Wrap any object with the GpuRoaring host fields (e.g. a downloaded GPU result)."""
    if isinstance(r, HostRoaring):
        return r
    return HostRoaring(keys=r.keys, types=r.types, offsets=r.offsets, cards=r.cards, n_containers=r.n_containers,
                       universe_size=r.universe_size, total_cardinality=r.total_cardinality,
                       bitmap_data=r.bitmap_data, n_bitmap_containers=r.n_bitmap_containers,
                       array_data=r.array_data, n_array_containers=r.n_array_containers,
                       array_pool_bytes=r.array_pool_bytes, run_data=r.run_data,
                       n_run_containers=r.n_run_containers, run_pool_bytes=r.run_pool_bytes,
                       key_index=r.key_index, max_key=r.max_key, negated=bool(r.negated))


def _check(rc: int, what: str):
    if rc != 0:
        raise RuntimeError(f"oracle {what} failed with code {rc}")


# ---- ref-semantics ------------------------------------------------------
def resolve_auto_threshold(universe: int, l2_bytes: int = DEFAULT_L2) -> int:
    return lib().orc_resolve_auto_threshold(universe, l2_bytes)


def upload_from_ids(ids, universe: int, threshold: int = PROMOTE_AUTO, l2_bytes: int = DEFAULT_L2) -> HostRoaring:
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    c = _OrcRoaring()
    _check(lib().orc_upload_from_ids(_ptr(ids), ids.size, universe, threshold, l2_bytes, C.byref(c)),
           "upload_from_ids")
    return _from_c(c)


def upload_from_bitset(words, universe: int) -> HostRoaring:
    words = np.ascontiguousarray(words, dtype=np.uint32)
    c = _OrcRoaring()
    _check(lib().orc_upload_from_bitset(_ptr(words), words.size, universe, C.byref(c)), "upload_from_bitset")
    return _from_c(c)


def set_operation(a: HostRoaring, b: HostRoaring, op: int) -> HostRoaring:
    c = _OrcRoaring()
    _check(lib().orc_set_operation(C.byref(a.as_c()), C.byref(b.as_c()), op, C.byref(c)), "set_operation")
    return _from_c(c)


def multi_and(inputs) -> HostRoaring:
    arr = (_OrcRoaring * max(1, len(inputs)))()
    for i, r in enumerate(inputs):
        arr[i] = r.as_c()
    c = _OrcRoaring()
    _check(lib().orc_multi_and(C.addressof(arr), len(inputs), C.byref(c)), "multi_and")
    return _from_c(c)


def contains_many(r: HostRoaring, ids) -> np.ndarray:
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    out = np.zeros(ids.size, dtype=np.uint32)
    lib().orc_contains_many(C.byref(as_host(r).as_c()), _ptr(ids), ids.size, _ptr(out))
    return out


def decompress(r: HostRoaring, n_words: Optional[int] = None) -> np.ndarray:
    if n_words is None:
        n_words = (r.universe_size + 31) // 32
    out = np.zeros(max(n_words, 1), dtype=np.uint32)
    lib().orc_decompress(C.byref(as_host(r).as_c()), _ptr(out), n_words)
    return out[:n_words]


def true_cardinality(r: HostRoaring) -> int:
    return lib().orc_true_cardinality(C.byref(as_host(r).as_c()))


def enumerate_ids(r) -> np.ndarray:
    """enumerate_ids (src/to_csr.cu:161-220): the stored ids as int64 (negation ignored)."""
    c = as_host(r).as_c()
    n = lib().orc_enumerate_ids(C.byref(c), None)
    out = np.zeros(max(n, 1), dtype=np.int64)
    lib().orc_enumerate_ids(C.byref(c), _ptr(out))
    return out[:n]


def promote_to_bitmap(r) -> HostRoaring:
    c = _OrcRoaring()
    _check(lib().orc_promote_to_bitmap(C.byref(as_host(r).as_c()), C.byref(c)), "promote_to_bitmap")
    return _from_c(c)


def deep_copy(r) -> HostRoaring:
    c = _OrcRoaring()
    _check(lib().orc_deep_copy(C.byref(as_host(r).as_c()), C.byref(c)), "deep_copy")
    return _from_c(c)


def promote_auto(r, l2_bytes: int = DEFAULT_L2) -> HostRoaring:
    """promote_auto (src/promote.cu:369-385): promote when AUTO resolves to ALL and a
    non-bitmap container exists, else a deep copy."""
    r = as_host(r)
    thr = lib().orc_resolve_auto_threshold(r.universe_size, l2_bytes)
    if thr == PROMOTE_ALL and (r.n_array_containers > 0 or r.n_run_containers > 0):
        return promote_to_bitmap(r)
    return deep_copy(r)


# ---- roaring-lite -------------------------------------------------------
class Lite:
    """Host Roaring (roaring-lite): stand-in for a CRoaring roaring_bitmap_t."""

    def __init__(self, handle):
        self.h = handle

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.rl_destroy(self.h)
            self.h = None

    @staticmethod
    def from_ids(ids) -> "Lite":
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        return Lite(lib().rl_from_ids(_ptr(ids), ids.size))

    @staticmethod
    def from_sorted_ids(ids) -> "Lite":
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        return Lite(lib().rl_from_sorted_ids(_ptr(ids), ids.size))

    @staticmethod
    def from_words(words) -> "Lite":
        """A flat bitset (u64 words, or u32 words reinterpreted; bit i = id i)."""
        w = np.ascontiguousarray(words)
        if w.dtype != np.uint64:
            w = np.ascontiguousarray(np.frombuffer(w.tobytes() + b"\0" * (-w.nbytes % 8), dtype=np.uint64))
        return Lite(lib().rl_from_words(_ptr(w), w.size))

    def copy(self) -> "Lite":
        return Lite(lib().rl_copy(self.h))

    def run_optimize(self) -> "Lite":
        lib().rl_run_optimize(self.h)
        return self

    def op(self, other: "Lite", op: int) -> "Lite":
        return Lite(lib().rl_op(self.h, other.h, op))

    def flip(self, lo: int, hi: int) -> "Lite":
        return Lite(lib().rl_flip(self.h, lo, hi))

    def contains(self, x: int) -> bool:
        return bool(lib().rl_contains(self.h, x))

    def contains_many(self, ids) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.zeros(ids.size, dtype=np.uint32)
        lib().rl_contains_many(self.h, _ptr(ids), ids.size, _ptr(out))
        return out

    def cardinality(self) -> int:
        return lib().rl_cardinality(self.h)

    def to_ids(self) -> np.ndarray:
        n = lib().rl_to_ids(self.h, None)
        out = np.zeros(max(n, 1), dtype=np.uint32)
        lib().rl_to_ids(self.h, _ptr(out))
        return out[:n]

    def n_containers(self) -> int:
        return lib().rl_n_containers(self.h)

    def portable_serialize(self) -> bytes:
        """The Roaring portable format (roaring_bitmap_portable_serialize's layout)."""
        n = lib().rl_portable_size(self.h)
        buf = np.zeros(max(n, 1), dtype=np.uint8)
        w = lib().rl_portable_serialize(self.h, _ptr(buf))
        assert w == n
        return buf[:n].tobytes()

    @staticmethod
    def portable_deserialize(data: bytes) -> "Lite":
        buf = np.frombuffer(bytes(data) + b"\0", dtype=np.uint8)
        used = C.c_uint64()
        h = lib().rl_portable_deserialize(_ptr(buf), len(data), C.byref(used))
        if not h:
            raise ValueError("not a well-formed portable Roaring bitmap")
        return Lite(h)

    def slice(self, key_lo: int, key_hi: int) -> "Lite":
        """The containers of keys [key_lo, key_hi), copied."""
        return Lite(lib().rl_slice(self.h, key_lo, key_hi))

    def shards(self, n: int, n_keys: int = 65536):
        """n slices over equal key ranges of [0, n_keys)."""
        step = (n_keys + n - 1) // n
        return [self.slice(i * step, min(n_keys, (i + 1) * step)) for i in range(n)]

    def type_counts(self):
        a, b, c = C.c_uint32(), C.c_uint32(), C.c_uint32()
        lib().rl_count_types(self.h, C.byref(a), C.byref(b), C.byref(c))
        return {"bitset": a.value, "array": b.value, "run": c.value}

    def containers(self):
        """(key, typecode, card, payload ndarray) per container; payload copied."""
        n = self.n_containers()
        arr = (_OrcContainer * max(1, n))()
        lib().rl_to_containers(self.h, C.addressof(arr))
        out = []
        for i in range(n):
            c = arr[i]
            if c.typecode == TC_BITSET:
                data = np.ctypeslib.as_array(C.cast(c.data, C.POINTER(C.c_uint64)), shape=(1024,)).copy()
            elif c.typecode == TC_ARRAY:
                data = np.ctypeslib.as_array(C.cast(c.data, C.POINTER(C.c_uint16)), shape=(max(c.card, 1),))[
                    :c.card].copy()
            else:
                data = np.ctypeslib.as_array(C.cast(c.data, C.POINTER(C.c_uint16)), shape=(max(2 * c.card, 1),))[
                    :2 * c.card].copy()
            out.append((c.key, c.typecode, c.card, data))
        return out


def upload_packed(bm: Lite, universe: Optional[int] = None, threshold: int = PROMOTE_AUTO,
                  l2_bytes: int = DEFAULT_L2) -> HostRoaring:
    """upload(roaring_bitmap_t*[, U], thr) -- src/upload.cpp:289-316."""
    src = bm
    complement = False
    logical = bm.cardinality()
    explicit_u = 0
    if universe is not None:
        explicit_u = universe
        if logical > universe // 2:  # :302
            src = bm.flip(0, universe)
            complement = True
    n = src.n_containers()
    arr = (_OrcContainer * max(1, n))()
    lib().rl_to_containers(src.h, C.addressof(arr))
    c = _OrcRoaring()
    _check(lib().orc_upload_packed(C.addressof(arr), n, explicit_u, 1 if complement else 0, logical, threshold,
                                   l2_bytes, C.byref(c)), "upload_packed")
    r = _from_c(c)
    del src
    return r


def upload_containers(containers, universe: int = 0, complemented: bool = False, logical: int = 0,
                      threshold: int = PROMOTE_AUTO, l2_bytes: int = DEFAULT_L2) -> HostRoaring:
    """upload_packed of host containers given as [(key, typecode, card | n_runs,
    payload)] sorted by key, taken as they are: the runs of a run container need
    not be sorted, disjoint or merged (src/upload.cpp:215-221 copies them as
    they are)."""
    arr = (_OrcContainer * max(1, len(containers)))()
    keep = []
    for i, (key, tc, card, payload) in enumerate(containers):
        p = np.ascontiguousarray(payload)
        keep.append(p)
        arr[i] = _OrcContainer(key, tc, card, p.ctypes.data if p.size else None)
    c = _OrcRoaring()
    _check(lib().orc_upload_packed(C.addressof(arr), len(containers), universe, 1 if complemented else 0, logical,
                                   threshold, l2_bytes, C.byref(c)), "upload_containers")
    del keep
    return _from_c(c)


# ---- generators ---------------------------------------------------------
def mt_bernoulli_ids(seed: int, density: float, universe: int) -> np.ndarray:
    out = np.zeros(max(universe, 1), dtype=np.uint32)
    n = C.c_uint64()
    lib().orc_mt_bernoulli_ids(seed, density, universe, _ptr(out), C.byref(n))
    return out[:n.value].copy()


def mt_raw(seed: int, n: int) -> np.ndarray:
    out = np.zeros(max(n, 1), dtype=np.uint32)
    lib().orc_mt_raw(seed, _ptr(out), n)
    return out[:n]


def splitmix64(x: int) -> int:
    return lib().orc_splitmix64(x)


def topk_bruteforce(base: np.ndarray, queries: np.ndarray, k: int, passing: Optional[np.ndarray] = None,
                    n_threads: int = 8):
    base = np.ascontiguousarray(base, dtype=np.float32)
    queries = np.ascontiguousarray(queries, dtype=np.float32)
    nq, dim = queries.shape
    dist = np.zeros((nq, k), dtype=np.float64)
    ids = np.zeros((nq, k), dtype=np.int64)
    p = None if passing is None else np.ascontiguousarray(passing, dtype=np.uint8)
    lib().orc_topk_bruteforce(_ptr(base), base.shape[0], _ptr(queries), nq, dim, _ptr(p) if p is not None else None,
                              k, _ptr(dist), _ptr(ids), n_threads)
    return dist, ids


# ---- CPU baselines (cpu_baseline.c): each returns (seconds of timed work, result) ----
def _handles(lites):
    arr = (C.c_void_p * max(1, len(lites)))(*[x.h for x in lites])
    return arr


def cpu_upload_ids(ids, universe: int, threads: int):
    """(seconds, HostRoaring) of the threaded bucket-build upload (all-bitmap layout)."""
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    c = _OrcRoaring()
    t = cpu_lib().orc_cpu_upload_ids(_ptr(ids), ids.size, universe, threads, C.byref(c))
    if t < 0:
        raise RuntimeError("orc_cpu_upload_ids: invalid input (key past max_key, or a complement)")
    return t, _from_c(c)


def cpu_setop(a_shards, b_shards, op: int, threads: int):
    """(seconds, total cardinality, containers) of rl_op over paired shards."""
    card, nc = C.c_uint64(), C.c_uint64()
    t = cpu_lib().orc_cpu_setop(_handles(a_shards), _handles(b_shards), len(a_shards), op, threads, C.byref(card),
                            C.byref(nc))
    return t, card.value, nc.value


def cpu_multi_and(input_shards, threads: int):
    """input_shards[j][s]: shard s of input j.  (seconds, cardinality, containers) of the AND chain."""
    k, n = len(input_shards), len(input_shards[0])
    flat = [x for shards in input_shards for x in shards]
    card, nc = C.c_uint64(), C.c_uint64()
    t = cpu_lib().orc_cpu_multi_and(_handles(flat), k, n, threads, C.byref(card), C.byref(nc))
    return t, card.value, nc.value


def cpu_contains(lite: "Lite", q, threads: int):
    q = np.ascontiguousarray(q, dtype=np.uint32)
    out = np.zeros(q.size, dtype=np.uint32)
    t = cpu_lib().orc_cpu_contains(lite.h, _ptr(q), q.size, _ptr(out), threads)
    return t, out


def cpu_config0(a_ids, b_ids, q):
    """(seconds total, [build, ops, queries] seconds, [AND, OR, ANDNOT, XOR] cards, hits)."""
    a = np.ascontiguousarray(a_ids, dtype=np.uint32)
    b = np.ascontiguousarray(b_ids, dtype=np.uint32)
    q = np.ascontiguousarray(q, dtype=np.uint32)
    parts = np.zeros(3, dtype=np.float64)
    cards = np.zeros(4, dtype=np.uint64)
    hits = C.c_uint64()
    t = cpu_lib().orc_cpu_config0(_ptr(a), a.size, _ptr(b), b.size, _ptr(q), q.size, _ptr(parts), _ptr(cards),
                              C.byref(hits))
    return t, parts.tolist(), [int(x) for x in cards], hits.value


def cpu_topk_fp32(base: np.ndarray, queries: np.ndarray, k: int, passing: Optional[np.ndarray], threads: int):
    """(seconds, dist fp32 [nq, k], ids int64 [nq, k]) of the blocked fp32 brute-force scan."""
    base = np.ascontiguousarray(base, dtype=np.float32)
    queries = np.ascontiguousarray(queries, dtype=np.float32)
    nq, dim = queries.shape
    dist = np.zeros((nq, k), dtype=np.float32)
    ids = np.zeros((nq, k), dtype=np.int64)
    p = None if passing is None else np.ascontiguousarray(passing, dtype=np.uint8)
    t = cpu_lib().orc_cpu_topk_fp32(_ptr(base), base.shape[0], _ptr(queries), nq, dim,
                                _ptr(p) if p is not None else None, k, _ptr(dist), _ptr(ids), threads)
    return t, dist, ids

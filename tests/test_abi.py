"""The C-ABI library loads on the CPU and exports every symbol the headers declare."""
import ctypes
import os
import re

import curoaring

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    src = open(os.path.join(ROOT, "include", "cu_roaring_abi.h")).read()
    return sorted(set(re.findall(r"^\s*(?:int|uint32_t|const char\*)\s+(cr_\w+)\s*\(", src, re.M)))


def test_header_declares_expected_entry_points():
    syms = _declared_symbols()
    for s in ("cr_upload_from_ids", "cr_set_operation", "cr_multi_and", "cr_contains_batch", "cr_free_async",
              "cr_resolve_auto_threshold", "cr_upload_containers", "cr_topk_filtered", "cr_decompress_to_bitset",
              "cr_enumerate_ids", "cr_promote_to_bitmap", "cr_promote_auto", "cr_deep_copy",
              "cr_portable_serialize", "cr_portable_deserialize", "cr_upload_batch", "cr_batch_multi_and"):
        assert s in syms
    assert set(syms) == set(curoaring.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = curoaring.load()
    for s in _declared_symbols():
        assert hasattr(lib, s), s


def test_struct_layout_matches_reference():
    # cu_roaring::GpuRoaring (types.cuh:15-54) on LP64: 120 bytes, negated at 108.
    assert ctypes.sizeof(curoaring.GpuRoaring) == 120
    assert curoaring.GpuRoaring.negated.offset == 108
    assert curoaring.GpuRoaring.key_index.offset == 96
    assert curoaring.GpuRoaring.total_cardinality.offset == 40
    # GpuRoaringView (roaring_view.cuh:14-37): 80 bytes, flags at 76/77.
    assert ctypes.sizeof(curoaring.GpuRoaringView) == 80
    assert curoaring.GpuRoaringView.all_bitmap.offset == 76
    # v2 GpuRoaringBatch (v2/include/cu_roaring_v2/types.cuh:37-86): 5 u32, 10 device and
    # 5 host pointers, 2 owners -> 160 bytes; GpuRoaringView (:95-107) 72 bytes.
    assert ctypes.sizeof(curoaring.RoaringBatch) == 160
    assert curoaring.RoaringBatch.container_starts.offset == 24
    assert curoaring.RoaringBatch.host_total_cardinalities.offset == 104
    assert ctypes.sizeof(curoaring.BatchView) == 72


def test_host_only_entry_points_without_gpu():
    # Calls that touch no device memory: argument validation and get_meta.
    lib = curoaring.load()
    out = curoaring.GpuRoaring()
    rc = lib.cr_set_operation(None, None, 0, None, ctypes.byref(out))
    assert rc == 2 and b"invalid" in lib.cr_last_error()
    m = curoaring.get_meta([(0, curoaring.TC_ARRAY, 3, __import__("numpy").array([1, 2, 3], dtype="uint16")),
                            (2, curoaring.TC_RUN, 1, __import__("numpy").array([0, 9], dtype="uint16"))])
    assert (m.n_containers, m.n_array_containers, m.n_run_containers, m.universe_size) == (2, 1, 1, 3 << 16)
    assert m.total_bytes == 2 * 9 + 3 * 2 + 1 * 4

"""The C++ drop-in surface end to end on the GPU: tests/cpp/api_check.cpp (built
by build()) calls the cu_roaring and cu_roaring::v2 host APIs and the
header-only device queries from kernels of its own, checking every result
against host truth from its input ids."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
pytestmark = pytest.mark.gpu


def test_cpp_api_end_to_end():
    exe = os.path.join(ROOT, "tests", "cpp", "api_check")
    assert os.path.exists(exe), "tests/cpp/api_check is built by __graft_entry__.build()"
    print("CASE cpp api_check", flush=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "api_check: OK" in r.stdout, r.stdout + r.stderr


def test_croaring_adapters():
    """The roaring_bitmap_t* overloads (upload(bm), upload(bm, U), get_meta(bm),
    v2::upload_batch) compiled with CU_ROARING_WITH_CROARING against the
    test-only CRoaring stand-in, byte-equal to the HostContainer path."""
    exe = os.path.join(ROOT, "tests", "cpp", "croaring_check")
    assert os.path.exists(exe), "tests/cpp/croaring_check is built by __graft_entry__.build()"
    print("CASE cpp croaring_check", flush=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=180)
    assert r.returncode == 0 and "croaring_check: OK" in r.stdout, r.stdout + r.stderr

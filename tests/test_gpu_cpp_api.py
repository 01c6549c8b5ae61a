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

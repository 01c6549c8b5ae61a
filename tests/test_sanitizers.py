"""Host code under AddressSanitizer + UndefinedBehaviorSanitizer (CPU only).

- The oracle (oracle/lib/liborc_sanitize.so, built by `make -C oracle`) runs the
  oracle's own test files in a child process with gcc's ASan runtime preloaded.
- The library's host C++ (host/api.cpp: the portable-format parser, the host
  complement of upload(bm, U), the C++ wrappers) runs in tests/cpp/host_sanitize
  (built by `make -C tests/cpp`), on portable bytes written here by roaring-lite
  and thousands of mutations of them.

Either fails on any sanitizer report (UBSan does not recover; ASan aborts).
"""
import os
import subprocess
import sys

import numpy as np
import pytest

import orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN_ENV = {"ASAN_OPTIONS": "detect_leaks=0:abort_on_error=1:allocator_may_return_null=1",
           "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1"}


def _libasan():
    try:
        p = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True,
                           timeout=30).stdout.strip()
    except (OSError, subprocess.SubprocessError):
        return None
    return p if p and os.path.isabs(p) and os.path.exists(p) else None


def test_oracle_under_sanitizers():
    lib = os.path.join(ROOT, "oracle", "lib", "liborc_sanitize.so")
    asan = _libasan()
    if not os.path.exists(lib) or asan is None:
        pytest.skip("sanitizer build of the oracle or gcc's libasan not available")
    files = sorted(f for f in os.listdir(os.path.join(ROOT, "tests")) if f.startswith("test_oracle_"))
    env = dict(os.environ, LD_PRELOAD=asan, ORC_LIB_PATH=lib, **SAN_ENV)
    # -s: a sanitizer report is written to the child's own stderr as it dies,
    # which pytest's capture would discard
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-s", "-p", "no:cacheprovider"] +
                       [os.path.join("tests", f) for f in files],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
    assert " passed" in out


def _cases(tmp):
    """Portable bytes of bitmaps with every container kind, and their sets."""
    rng = np.random.default_rng(77)
    sets = []
    sets.append((0, np.unique(rng.integers(0, 1 << 20, 3000, dtype=np.uint64)).astype(np.uint32)))  # arrays
    sets.append((1 << 20, np.nonzero(rng.random(1 << 20) < 0.3)[0].astype(np.uint32)))  # bitsets
    runs = np.concatenate([np.arange(s, s + int(rng.integers(1, 5000))) for s in range(0, 1 << 21, 9000)])
    sets.append((0, np.unique(runs).astype(np.uint32)))  # run containers after run_optimize
    dense = np.nonzero(rng.random(300003) < 0.8)[0].astype(np.uint32)
    sets.append((300003, dense))  # more than U/2: the complement is stored (odd U)
    sets.append((200000, np.concatenate([np.arange(0, 150000), np.arange(150100, 200000)]).astype(np.uint32)))
    sets.append((70000, np.array([0, 65535, 65536, 69999], dtype=np.uint32)))
    for i, (u, ids) in enumerate(sets):
        lite = orc.Lite.from_sorted_ids(ids)
        if i != 1:
            lite = lite.run_optimize()
        with open(os.path.join(tmp, f"case_{i}.bin"), "wb") as f:
            f.write(lite.portable_serialize())
        with open(os.path.join(tmp, f"case_{i}.ids"), "wb") as f:
            f.write(np.uint32(u).tobytes() + ids.astype(np.uint32).tobytes())
    return len(sets)


def test_host_layer_under_sanitizers(tmp_path):
    exe = os.path.join(ROOT, "tests", "cpp", "host_sanitize")
    if not os.path.exists(exe):
        pytest.skip("tests/cpp/host_sanitize is built by __graft_entry__.build()")
    n = _cases(str(tmp_path))
    r = subprocess.run([exe, str(tmp_path)], capture_output=True, text=True, timeout=600,
                       env=dict(os.environ, **SAN_ENV))
    out = r.stdout + r.stderr
    assert r.returncode == 0 and "host_sanitize: OK" in out, out[-4000:]
    assert f"({n} cases" in out

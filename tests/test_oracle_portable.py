"""The oracle's Roaring portable-format writer and reader (CPU).

The expected byte strings are assembled here with struct from the format
specification (RoaringFormatSpec): cookie 12346 + u32 size without run
containers, else u16 12347 + u16 size-1 + run-flag bytes; (key, card-1) pairs;
u32 offsets from the stream start iff there is no run container or size >= 4;
then run (u16 n_runs + (start, length-1) pairs), array (u16 values) or bitset
(1024 u64) payloads.
"""
import struct

import numpy as np
import pytest

import orc


def _lite(ids, optimize):
    lite = orc.Lite.from_sorted_ids(np.asarray(ids, dtype=np.uint32))
    return lite.run_optimize() if optimize else lite


def test_array_without_runs():
    want = struct.pack("<II", 12346, 1) + struct.pack("<HH", 0, 2) + struct.pack("<I", 16) + struct.pack("<HHH", 1, 2, 3)
    assert _lite([1, 2, 3], False).portable_serialize() == want
    assert list(orc.Lite.portable_deserialize(want).to_ids()) == [1, 2, 3]


def test_single_run_has_no_offset_header():
    want = struct.pack("<HH", 12347, 0) + bytes([1]) + struct.pack("<HH", 0, 2) + struct.pack("<H", 1) + \
        struct.pack("<HH", 1, 2)
    assert _lite([1, 2, 3], True).portable_serialize() == want
    assert list(orc.Lite.portable_deserialize(want).to_ids()) == [1, 2, 3]


def _five_container_case():
    ids = np.concatenate([
        np.arange(10, 20),                      # key 0: run [10, 19]
        [65536 + 5],                            # key 1: array {5}
        2 * 65536 + np.arange(0, 10000, 2),     # key 2: 5000 values -> bitset
        [3 * 65536, 3 * 65536 + 65535],         # key 3: array {0, 65535}
        4 * 65536 + np.arange(65536),           # key 4: full -> run [0, 65535]
    ]).astype(np.uint32)
    hdr = struct.pack("<HH", 12347, 4) + bytes([0b00010001])
    hdr += b"".join(struct.pack("<HH", k, c - 1) for k, c in ((0, 10), (1, 1), (2, 5000), (3, 2), (4, 65536)))
    sizes = [2 + 4, 2, 8192, 4, 2 + 4]
    off = 4 + 1 + 5 * 4 + 5 * 4
    offs = []
    for s in sizes:
        offs.append(off)
        off += s
    hdr += struct.pack("<5I", *offs)
    words = np.zeros(1024, dtype=np.uint64)
    for v in range(0, 10000, 2):
        words[v // 64] |= np.uint64(1) << np.uint64(v % 64)
    body = struct.pack("<HHH", 1, 10, 9) + struct.pack("<H", 5) + words.astype("<u8").tobytes() + \
        struct.pack("<HH", 0, 65535) + struct.pack("<HHH", 1, 0, 65535)
    return ids, hdr + body


def test_five_containers_with_runs_and_offsets():
    ids, want = _five_container_case()
    assert len(want) == 8255
    lite = _lite(ids, True)
    assert lite.type_counts() == {"bitset": 1, "array": 2, "run": 2}
    assert lite.portable_serialize() == want
    back = orc.Lite.portable_deserialize(want)
    assert np.array_equal(back.to_ids(), ids)
    assert back.portable_serialize() == want


def test_empty_and_bitset_without_runs():
    assert _lite([], False).portable_serialize() == struct.pack("<II", 12346, 0)
    assert orc.Lite.portable_deserialize(struct.pack("<II", 12346, 0)).cardinality() == 0
    ids = 7 * 65536 + np.arange(4097)
    words = np.zeros(1024, dtype=np.uint64)
    words[:64] = np.uint64(0xFFFFFFFFFFFFFFFF)
    words[64] = 1
    want = struct.pack("<II", 12346, 1) + struct.pack("<HH", 7, 4096) + struct.pack("<I", 16) + \
        words.astype("<u8").tobytes()
    assert _lite(ids, False).portable_serialize() == want
    assert np.array_equal(orc.Lite.portable_deserialize(want).to_ids(), ids)


def test_malformed_inputs_are_rejected():
    _, good = _five_container_case()
    for cut in (0, 3, 5, 20, 44, 50, 52, 100, 8244, 8254):
        with pytest.raises(ValueError):
            orc.Lite.portable_deserialize(good[:cut])
    with pytest.raises(ValueError):
        orc.Lite.portable_deserialize(struct.pack("<II", 12345, 0))
    unordered = struct.pack("<II", 12346, 2) + struct.pack("<HHHH", 5, 0, 3, 0) + struct.pack("<II", 24, 26) + \
        struct.pack("<HH", 1, 1)
    with pytest.raises(ValueError):
        orc.Lite.portable_deserialize(unordered)
    past_end = struct.pack("<HH", 12347, 0) + bytes([1]) + struct.pack("<HH", 0, 9) + struct.pack("<HHH", 1, 65530, 9)
    with pytest.raises(ValueError):
        orc.Lite.portable_deserialize(past_end)


@pytest.mark.parametrize("seed", range(6))
def test_random_round_trips(seed):
    rng = np.random.default_rng(seed)
    parts = []
    for key in range(int(rng.integers(1, 30))):
        kind = int(rng.integers(0, 4))
        base = int(rng.integers(0, 65536)) * 65536 if seed % 2 else key * 65536
        if kind == 0:
            parts.append(base + np.unique(rng.integers(0, 65536, int(rng.integers(1, 5000)))))
        elif kind == 1:
            parts.append(base + np.nonzero(rng.random(65536) < rng.uniform(0.05, 0.95))[0])
        elif kind == 2:
            s = int(rng.integers(0, 60000))
            parts.append(base + np.arange(s, s + int(rng.integers(1, 65536 - s))))
    ids = np.unique(np.concatenate(parts) if parts else np.zeros(0)).astype(np.uint32)
    for opt in (False, True):
        lite = _lite(ids, opt)
        data = lite.portable_serialize()
        back = orc.Lite.portable_deserialize(data)
        assert np.array_equal(back.to_ids(), ids)
        assert back.portable_serialize() == data

"""cr_portable_deserialize rejects malformed input in its host-side parse,
before any device work, so these run without a GPU."""
import struct

import numpy as np
import pytest

import curoaring
import orc


def _good():
    ids = np.concatenate([np.arange(10, 20), [65536 + 5], 2 * 65536 + np.arange(0, 10000, 2),
                          [3 * 65536, 3 * 65536 + 65535], 4 * 65536 + np.arange(65536)]).astype(np.uint32)
    return orc.Lite.from_sorted_ids(ids).run_optimize().portable_serialize()


@pytest.mark.parametrize("cut", [0, 3, 5, 20, 44, 50, 52, 100, 8244, 8254])
def test_truncated(cut):
    data = _good()
    assert len(data) == 8255
    with pytest.raises(curoaring.CrError) as e:
        curoaring.portable_deserialize(data[:cut])
    assert e.value.code == curoaring.CR_ERR_INVALID


@pytest.mark.parametrize("data,why", [
    (struct.pack("<II", 12345, 0), "unknown cookie"),
    (struct.pack("<II", 12346, 70000), "more than 65536"),
    (struct.pack("<II", 12346, 2) + struct.pack("<HHHH", 5, 0, 3, 0) + struct.pack("<II", 24, 26) +
     struct.pack("<HH", 1, 1), "keys not strictly increasing"),
    (struct.pack("<HH", 12347, 0) + bytes([1]) + struct.pack("<HH", 0, 9) + struct.pack("<HHH", 1, 65530, 9),
     "run past"),
])
def test_malformed(data, why):
    with pytest.raises(curoaring.CrError) as e:
        curoaring.portable_deserialize(data)
    assert e.value.code == curoaring.CR_ERR_INVALID and why in str(e.value)

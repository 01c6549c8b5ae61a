"""Shared test helpers: truth construction, canonical dumps, reference-test inputs."""
from __future__ import annotations

import numpy as np

import orc


def auto_l2(gpu) -> int:
    """The L2 size for which the reference's PROMOTE_AUTO rule (2 ceil(U/8) > L2,
    which the oracle restates) gives the library's gfx950 verdicts
    (32 ceil(U/8) > one XCD's L2): that L2 / 16."""
    return gpu.device_l2_bytes() // 16


def flat_from_ids(ids, universe: int, n_words=None) -> np.ndarray:
    """Independent truth: a flat uint32 bitset with bit i set for each id < 32*n_words."""
    if n_words is None:
        n_words = (universe + 31) // 32
    ids = np.asarray(ids, dtype=np.uint64)
    ids = ids[ids < 32 * n_words]
    bits = np.zeros(32 * n_words, dtype=bool)
    bits[ids] = True
    return np.packbits(bits.reshape(-1, 8), axis=1, bitorder="little").reshape(-1).view(np.uint32).copy()


def ids_from_flat(words: np.ndarray) -> np.ndarray:
    bits = np.unpackbits(words.view(np.uint8), bitorder="little")
    return np.nonzero(bits)[0].astype(np.uint32)


def words_mask(words: np.ndarray, universe: int) -> np.ndarray:
    w = words.copy()
    n_full = universe // 32
    tail = universe % 32
    if tail and n_full < w.size:
        w[n_full] &= np.uint32((1 << tail) - 1)
        w[n_full + 1:] = 0
    elif not tail:
        w[n_full:] = 0
    return w


def container_payload(r, i: int) -> bytes:
    t = int(r.types[i])
    off = int(r.offsets[i])
    card = int(r.cards[i])
    if t == orc.BITMAP:
        w = off // 8
        return r.bitmap_data[w:w + 1024].tobytes()
    if t == orc.ARRAY:
        e = off // 2
        return r.array_data[e:e + card].tobytes()
    e = off // 2
    return r.run_data[e:e + 2 * card].tobytes()


def canonical(r, strict: bool = False) -> dict:
    """Parity serialisation: header + per-container (key, type, card, payload).

    Pool holes and offsets are compared only with strict=True.
    """
    d = {
        "n_containers": int(r.n_containers),
        "universe_size": int(r.universe_size),
        "negated": bool(r.negated),
        "total_cardinality": int(r.total_cardinality),
        "max_key": int(r.max_key),
        "has_key_index": r.key_index is not None,
        "n_bitmap": int(r.n_bitmap_containers),
        "n_array": int(r.n_array_containers),
        "n_run": int(r.n_run_containers),
        "array_pool_bytes": int(r.array_pool_bytes),
        "run_pool_bytes": int(r.run_pool_bytes),
    }
    conts = []
    for i in range(int(r.n_containers)):
        conts.append((int(r.keys[i]), int(r.types[i]), int(r.cards[i]), container_payload(r, i)))
    d["containers"] = conts
    if r.key_index is not None:
        d["key_index"] = r.key_index.tobytes()
    if strict:
        d["offsets"] = r.offsets[: r.n_containers].tobytes()
        d["bitmap_pool_words"] = int(r.bitmap_data.size)
    return d


def assert_same(got, want, strict: bool = False, what: str = ""):
    g, w = canonical(got, strict), canonical(want, strict)
    for k in w:
        if k == "containers":
            continue
        assert g[k] == w[k], f"{what}: field {k} differs: got {g[k]!r} want {w[k]!r}"
    assert len(g["containers"]) == len(w["containers"])
    for i, (gc, wc) in enumerate(zip(g["containers"], w["containers"])):
        assert gc[:3] == wc[:3], f"{what}: container {i} header got {gc[:3]} want {wc[:3]}"
        assert gc[3] == wc[3], f"{what}: container {i} (key {wc[0]}) payload differs"


# ---- reference-test input generators (std::mt19937 based) ---------------
def assert_packed_offsets(h, what: str = ""):
    """The packed layout's offsets, checked against what the layout itself fixes:
    containers go into their type's pool in key order, back to back, so each
    offset is the sum of the sizes of the earlier containers of its type --
    8192 bytes a bitmap, 2 bytes a value of an array, 4 bytes a run
    (src/upload.cpp:89-287) -- and each pool holds exactly its containers."""
    n = h.n_containers
    types, cards, offs = np.asarray(h.types[:n]), np.asarray(h.cards[:n]).astype(np.int64), np.asarray(h.offsets[:n])
    keys = np.asarray(h.keys[:n]).astype(np.int64)
    assert np.all(np.diff(keys) > 0), f"{what}: keys not ascending"
    size = np.where(types == 1, 8192, np.where(types == 0, 2 * cards, 4 * cards))
    for ty, pool in ((1, "bitmap"), (0, "array"), (2, "run")):
        m = types == ty
        want = np.concatenate([[0], np.cumsum(size[m])[:-1]]) if m.any() else np.zeros(0, np.int64)
        assert np.array_equal(offs[m].astype(np.int64), want), f"{what}: {pool} offsets are not the prefix sums"
    assert 8192 * int((types == 1).sum()) == 8192 * h.n_bitmap_containers
    assert int(size[types == 0].sum()) == h.array_pool_bytes, f"{what}: array pool size"
    assert int(size[types == 2].sum()) == h.run_pool_bytes, f"{what}: run pool size"


def mt_bernoulli(seed: int, density: float, universe: int) -> np.ndarray:
    """ids i < universe with uniform_real_distribution<double>(0,1)(mt19937(seed)) < density."""
    return orc.mt_bernoulli_ids(seed, density, universe)


def mt_mod_filter(seed: int, universe: int, mod: int, keep_zero: bool) -> np.ndarray:
    """ids with (gen() % mod == 0) (keep_zero) or (!= 0) -- test/test_complement.cu style."""
    g = orc.mt_raw(seed, universe)
    m = (g % mod) == 0
    return np.nonzero(m if keep_zero else ~m)[0].astype(np.uint32)


def mt_low16_density(gen_values: np.ndarray, density: float) -> np.ndarray:
    return (gen_values & 0xFFFF) < np.uint32(int(density * 65536.0))

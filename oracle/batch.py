"""CPU restatement of the reference's v2 batch API (TEST INFRASTRUCTURE ONLY).

Only tests/ may use this module, as the checker.  Each function follows the
reference file:line it cites, on host containers as roaring-lite (or
CRoaring's high_low_container) lists them: (key, typecode, card|n_runs, data)
with typecode 1 bitset / 2 array / 3 run.

Pinning (tests/test_oracle_batch.py): the assertions of the reference's own
v2 test (v2/test/test_basic.cu:143-430) on its mixed inputs, re-derived with
roaring-lite as the CRoaring stand-in (cardinalities, slice widths, contains
on the probe set, multi_and of {0,1,2} and {2,3} against lite AND, the
all-bitmap rejection, decompress per id), plus flat-bitset brute force on
random batches.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np

ARRAY, BITMAP, RUN = 0, 1, 2          # v2/include/cu_roaring_v2/types.cuh:7-11
TC_BITSET, TC_ARRAY, TC_RUN = 1, 2, 3  # CRoaring typecodes (v2/src/upload.cpp:25-27)


@dataclass
class HostBatch:
    """GpuRoaringBatch (v2/include/cu_roaring_v2/types.cuh:37-86), host copy."""
    n_bitmaps: int = 0
    total_containers: int = 0
    n_bitmap_containers_total: int = 0
    array_pool_bytes: int = 0
    run_pool_bytes: int = 0
    container_starts: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint32))
    key_index_starts: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint32))
    keys: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint16))
    types: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint8))
    offsets: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint32))
    cards: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint16))
    key_indices: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint16))
    bitmap_data: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint64))
    array_data: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint16))
    run_data: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint16))
    host_total_cardinalities: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint64))
    host_universe_sizes: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint32))
    host_container_starts: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint32))
    host_key_index_starts: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint32))
    host_n_bitmap_containers: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint32))


def _true_card(tc, card, data) -> int:
    if tc == TC_RUN:
        return int(np.sum(data[1::2].astype(np.int64) + 1))
    return int(card)


def upload_batch(bitmaps: Sequence[list]) -> HostBatch:
    """upload_batch (v2/src/upload.cpp:45-259, 319-360): container types kept,
    CSR starts, per-type pools packed in global container order, byte offsets,
    key_indices 0xFFFF except present keys (LOCAL index), a bitset card > 65535
    or < 0 stored as 0, a run card = n_runs; host mirrors: total cardinality,
    universe (max_key + 1) << 16 (u32), starts, bitset counts."""
    n = len(bitmaps)
    if n == 0:
        return HostBatch()
    B = HostBatch(n_bitmaps=n)
    cs, ks = [0], [0]
    keys, types, offs, cards = [], [], [], []
    kidx_parts, bmp, arr, run = [], [], [], []
    tot_card, universe, nbm = [], [], []
    bmp_cur = arr_cur = run_cur = 0
    for conts in bitmaps:
        nc = len(conts)
        klen = (int(conts[-1][0]) + 1) if nc else 0
        ki = np.full(klen, 0xFFFF, np.uint16)
        tcard, nb = 0, 0
        for i, (key, tc, card, data) in enumerate(conts):
            if tc not in (TC_BITSET, TC_ARRAY, TC_RUN):
                raise ValueError(f"unknown typecode {tc}")
            keys.append(key)
            ki[key] = i
            tcard += _true_card(tc, card, data)
            if tc == TC_BITSET:
                nb += 1
                types.append(BITMAP)
                offs.append(bmp_cur * 8)
                cards.append(0 if (card > 65535 or card < 0) else card)
                bmp.append(np.asarray(data, np.uint64))
                bmp_cur += 1024
            elif tc == TC_ARRAY:
                types.append(ARRAY)
                offs.append(arr_cur * 2)
                cards.append(card)
                arr.append(np.asarray(data, np.uint16))
                arr_cur += card
            else:
                types.append(RUN)
                offs.append(run_cur * 4)
                cards.append(card)
                run.append(np.asarray(data, np.uint16))
                run_cur += card
        cs.append(cs[-1] + nc)
        ks.append(ks[-1] + klen)
        kidx_parts.append(ki)
        tot_card.append(tcard)
        universe.append((klen << 16) & 0xFFFFFFFF if nc else 0)
        nbm.append(nb)
    B.total_containers = cs[-1]
    B.n_bitmap_containers_total = int(sum(nbm))
    B.array_pool_bytes = arr_cur * 2
    B.run_pool_bytes = run_cur * 4
    B.container_starts = np.array(cs, np.uint32)
    B.key_index_starts = np.array(ks, np.uint32)
    B.keys = np.array(keys, np.uint16)
    B.types = np.array(types, np.uint8)
    B.offsets = np.array(offs, np.uint32)
    B.cards = np.array(cards, np.uint16)
    B.key_indices = np.concatenate(kidx_parts) if kidx_parts else np.zeros(0, np.uint16)
    B.bitmap_data = np.concatenate(bmp) if bmp else np.zeros(0, np.uint64)
    B.array_data = np.concatenate(arr) if arr else np.zeros(0, np.uint16)
    B.run_data = np.concatenate(run) if run else np.zeros(0, np.uint16)
    B.host_total_cardinalities = np.array(tot_card, np.uint64)
    B.host_universe_sizes = np.array(universe, np.uint32)
    B.host_container_starts = B.container_starts.copy()
    B.host_key_index_starts = B.key_index_starts.copy()
    B.host_n_bitmap_containers = np.array(nbm, np.uint32)
    return B


def container_image(B: HostBatch, cid: int) -> np.ndarray:
    """The 1024-word bitset of global container cid (runs clamped at 0xFFFF,
    v2/src/promote.cu:103-106)."""
    t, off, card = int(B.types[cid]), int(B.offsets[cid]), int(B.cards[cid])
    if t == BITMAP:
        return B.bitmap_data[off // 8: off // 8 + 1024].copy()
    bits = np.zeros(65536, bool)
    if t == ARRAY:
        bits[B.array_data[off // 2: off // 2 + card]] = True
    else:
        r = B.run_data[off // 2: off // 2 + 2 * card].astype(np.int64)
        for s, l in zip(r[0::2], r[1::2]):
            bits[s: min(0xFFFF, s + l) + 1] = True
    return np.packbits(bits, bitorder="little").view(np.uint64).copy()


def _popc(words: np.ndarray) -> int:
    return int(np.bitwise_count(words).sum(dtype=np.int64))


def promote_batch(B: HostBatch) -> HostBatch:
    """promote_batch (v2/src/promote.cu:28-304): every container a BITMAP at
    offset cid * 8192, card = popcount (65536 stored as 0); starts, keys and
    key_indices copied; host n_bitmap[b] = n_containers of b."""
    if B.n_bitmaps == 0:
        return HostBatch()
    n, T = B.n_bitmaps, B.total_containers
    P = HostBatch(n_bitmaps=n, total_containers=T, n_bitmap_containers_total=T)
    P.container_starts, P.key_index_starts = B.container_starts.copy(), B.key_index_starts.copy()
    P.keys, P.key_indices = B.keys.copy(), B.key_indices.copy()
    imgs = [container_image(B, c) for c in range(T)]
    P.types = np.full(T, BITMAP, np.uint8)
    P.offsets = (np.arange(T, dtype=np.uint32) * 8192).astype(np.uint32)
    P.cards = np.array([(lambda v: 0 if v > 65535 else v)(_popc(w)) for w in imgs], np.uint16)
    P.bitmap_data = np.concatenate(imgs) if imgs else np.zeros(0, np.uint64)
    P.host_total_cardinalities = B.host_total_cardinalities.copy()
    P.host_universe_sizes = B.host_universe_sizes.copy()
    P.host_container_starts = B.host_container_starts.copy()
    P.host_key_index_starts = B.host_key_index_starts.copy()
    P.host_n_bitmap_containers = np.diff(B.host_container_starts).astype(np.uint32)
    return P


def _empty_one_batch() -> HostBatch:
    """v2/src/multi_and.cu:207-242: one empty bitmap, CSR starts all zero."""
    E = HostBatch(n_bitmaps=1)
    E.container_starts = np.zeros(2, np.uint32)
    E.key_index_starts = np.zeros(2, np.uint32)
    E.host_total_cardinalities = np.zeros(1, np.uint64)
    E.host_universe_sizes = np.zeros(1, np.uint32)
    E.host_container_starts = np.zeros(2, np.uint32)
    E.host_key_index_starts = np.zeros(2, np.uint32)
    E.host_n_bitmap_containers = np.zeros(1, np.uint32)
    return E


def multi_and(B: HostBatch, indices: Sequence[int]) -> HostBatch:
    """multi_and (v2/src/multi_and.cu:244-470).  Inputs must be all-bitmap
    (ValueError otherwise); any empty input gives the empty 1-batch; the anchor
    is the first input of fewest containers; an anchor key survives iff every
    other input's key_indices has it (zero-card results are kept); the output
    is in anchor order, BITMAP at k * 8192, card = popcount (65536 as 0), its
    key_indices sized like the anchor's; universe = anchor kidx len << 16."""
    indices = [int(i) for i in indices]
    if not indices:
        raise ValueError("n_inputs must be >= 1")
    hs = B.host_container_starts
    for b in indices:
        if b >= B.n_bitmaps:
            raise IndexError(b)
        if int(B.host_n_bitmap_containers[b]) != int(hs[b + 1] - hs[b]):
            raise ValueError(f"bitmap {b} has non-bitmap containers")
    if any(hs[b + 1] == hs[b] for b in indices):
        return _empty_one_batch()
    sizes = [int(hs[b + 1] - hs[b]) for b in indices]
    ap = int(np.argmin(sizes))
    ab = indices[ap]
    a0, an = int(hs[ab]), sizes[ap]
    klen = int(B.host_key_index_starts[ab + 1] - B.host_key_index_starts[ab])
    out_keys, imgs = [], []
    for i in range(an):
        key = int(B.keys[a0 + i])
        ok = True
        for b in indices:
            if b == ab:
                continue
            k0, k1 = int(B.key_index_starts[b]), int(B.key_index_starts[b + 1])
            if key >= k1 - k0 or B.key_indices[k0 + key] == 0xFFFF:
                ok = False
                break
        if not ok:
            continue
        acc = np.full(1024, np.uint64(0xFFFFFFFFFFFFFFFF), np.uint64)
        for b in indices:
            k0 = int(B.key_index_starts[b])
            cid = int(B.container_starts[b]) + int(B.key_indices[k0 + key])
            acc &= B.bitmap_data[int(B.offsets[cid]) // 8: int(B.offsets[cid]) // 8 + 1024]
        out_keys.append(key)
        imgs.append(acc)
    m = len(out_keys)
    R = HostBatch(n_bitmaps=1, total_containers=m, n_bitmap_containers_total=m)
    R.container_starts = np.array([0, m], np.uint32)
    R.key_index_starts = np.array([0, klen], np.uint32)
    R.keys = np.array(out_keys, np.uint16)
    R.types = np.full(m, BITMAP, np.uint8)
    R.offsets = (np.arange(m, dtype=np.uint32) * 8192).astype(np.uint32)
    pcs = [_popc(w) for w in imgs]
    R.cards = np.array([0 if v > 65535 else v for v in pcs], np.uint16)
    R.key_indices = np.full(klen, 0xFFFF, np.uint16)
    for k, key in enumerate(out_keys):
        R.key_indices[key] = k
    R.bitmap_data = np.concatenate(imgs) if imgs else np.zeros(0, np.uint64)
    R.host_total_cardinalities = np.array([sum(pcs)], np.uint64)
    R.host_universe_sizes = np.array([(klen << 16) & 0xFFFFFFFF], np.uint32)
    R.host_container_starts = R.container_starts.copy()
    R.host_key_index_starts = R.key_index_starts.copy()
    R.host_n_bitmap_containers = np.array([m], np.uint32)
    return R


def decompress_batch(B: HostBatch, words_each: int, prior: Optional[np.ndarray] = None) -> np.ndarray:
    """decompress_batch (v2/src/decompress.cu:42-178): bitmap b's container
    windows at b * words_each + key * 1024, clipped to the slot; a BITMAP
    window is stored, an ARRAY / RUN window is OR-ed into what the buffer held.
    ValueError when words_each < ceil(max host universe / 64)."""
    out = np.zeros(B.n_bitmaps * words_each, np.uint64) if prior is None else prior.copy()
    if B.n_bitmaps == 0 or B.total_containers == 0:
        return out
    need = (int(B.host_universe_sizes.max()) + 63) // 64
    if words_each < need:
        raise ValueError("words_each too small")
    for b in range(B.n_bitmaps):
        base, end = b * words_each, (b + 1) * words_each
        for cid in range(int(B.container_starts[b]), int(B.container_starts[b + 1])):
            wb = base + int(B.keys[cid]) * 1024
            if wb >= end:
                continue
            win = min(1024, end - wb)
            img = container_image(B, cid)[:win]
            if int(B.types[cid]) == BITMAP:
                out[wb: wb + win] = img
            else:
                out[wb: wb + win] |= img
    return out


def _contains_in(B: HostBatch, cid: int, low: int) -> bool:
    """v2/include/cu_roaring_v2/query.cuh:15-66."""
    t, off, card = int(B.types[cid]), int(B.offsets[cid]), int(B.cards[cid])
    if t == BITMAP:
        return bool((int(B.bitmap_data[off // 8 + (low >> 6)]) >> (low & 63)) & 1)
    if t == ARRAY:
        a = B.array_data[off // 2: off // 2 + card]
        i = int(np.searchsorted(a, low))
        return i < card and int(a[i]) == low
    r = B.run_data[off // 2: off // 2 + 2 * card].astype(np.int64)
    i = int(np.searchsorted(r[0::2], low, side="right"))
    return i > 0 and low <= int(r[2 * (i - 1)]) + int(r[2 * (i - 1) + 1])


def contains(B: HostBatch, b: int, ids) -> np.ndarray:
    """contains(batch, b, id) (query.cuh:97-112)."""
    out = np.zeros(len(ids), np.uint8)
    if b >= B.n_bitmaps:
        return out
    k0, k1 = int(B.key_index_starts[b]), int(B.key_index_starts[b + 1])
    c0 = int(B.container_starts[b])
    for j, x in enumerate(np.asarray(ids, np.uint64)):
        hi, lo = int(x) >> 16, int(x) & 0xFFFF
        if hi >= k1 - k0:
            continue
        loc = int(B.key_indices[k0 + hi])
        if loc != 0xFFFF:
            out[j] = _contains_in(B, c0 + loc, lo)
    return out


def view_contains(B: HostBatch, b: int, ids) -> np.ndarray:
    """contains(make_view(batch, b), id) (query.cuh:75-92; v2/src/upload.cpp:383-415):
    an empty slice answers false, a key above max_key (= kidx len - 1) false."""
    out = np.zeros(len(ids), np.uint8)
    n_c = int(B.host_container_starts[b + 1] - B.host_container_starts[b])
    if n_c == 0:
        return out
    k0, k1 = int(B.host_key_index_starts[b]), int(B.host_key_index_starts[b + 1])
    max_key = k1 - k0 - 1 if k1 > k0 else 0
    c0 = int(B.host_container_starts[b])
    for j, x in enumerate(np.asarray(ids, np.uint64)):
        hi, lo = int(x) >> 16, int(x) & 0xFFFF
        if hi > max_key:
            continue
        loc = int(B.key_indices[k0 + hi])
        if loc != 0xFFFF:
            out[j] = _contains_in(B, c0 + loc, lo)
    return out

"""GPU checks at the benchmark's full sizes (universe 2^30), through properties
that do not need the CPU oracle: every result is decoded back to a flat
bitset on the device and compared with the same set built independently by
torch (index_add of distinct bits, bitwise ops on words), plus the metadata
the reference fixes for an all-bitmap result (src/upload_ids.cu:171-295).

Inputs come from bench.py's generators, so these are the configurations the
bench line is measured on and the set-operation and
multi_and configs over 2^30.
"""
import pytest

import bench
import orc

pytestmark = pytest.mark.gpu

U = 1 << 30
NW = U // 32


def _say(*a):
    print("CASE", *a, flush=True)


@pytest.fixture(scope="module")
def torch():
    import torch as t
    return t


def _bitset_of_ids(torch, ids):
    """Flat 2^30-bit bitset (int32 words) of an int32 id tensor: the distinct ids'
    bits summed per word (distinct bits, so the sum is the OR)."""
    u = torch.unique(ids.to(torch.int64))
    w = torch.zeros(NW, device=ids.device, dtype=torch.int64)
    w.index_add_(0, u >> 5, torch.ones_like(u) << (u & 31))
    return (w - (w >= (1 << 31)).to(torch.int64) * (1 << 32)).to(torch.int32), int(u.numel())


def _decoded(torch, cr, g):
    out = torch.empty(NW, device="cuda", dtype=torch.int32)
    cr.decompress_to_bitset(g, out)
    torch.cuda.synchronize()
    return out


def _popcount_words(torch, w):
    x = w.to(torch.int64) & 0xFFFFFFFF
    c = torch.zeros_like(x)
    for s in range(32):
        c += (x >> s) & 1
    return c


def _check_all_bitmap_ids_result(torch, cr, g, want_words, n_distinct):
    """Metadata of upload_from_ids' GPU path: all-BITMAP, keys ascending,
    offsets i*8192, cards = popcount with 65536 stored as 0, key_index over
    [0, max_key], max_key = (U-1)>>16, total = distinct ids, not negated."""
    h = cr.download(g)
    assert not h.negated and h.universe_size == U and h.max_key == (U - 1) >> 16
    assert h.total_cardinality == n_distinct
    per_key = _popcount_words(torch, want_words).view(-1, 2048).sum(dim=1).cpu().numpy()
    present = per_key.nonzero()[0]
    assert h.n_containers == len(present) == h.n_bitmap_containers
    assert (h.keys[: len(present)] == present).all()
    assert (h.types[: len(present)] == 1).all()  # BITMAP (types.cuh ContainerType)
    assert (h.offsets[: len(present)] == (8192 * torch.arange(len(present)).numpy()).astype("uint32")).all()
    assert (h.cards[: len(present)] == (per_key[present] % 65536)).all()
    ki = h.key_index
    assert (ki[present] == torch.arange(len(present)).numpy()).all()
    absent = (per_key == 0).nonzero()[0]
    assert (ki[absent] == 0xFFFF).all()


@pytest.mark.parametrize("kind", ["uniform", "clustered"])
def test_upload_from_ids_full_size(gpu, torch, kind):
    """100M ids over 2^30, uniform (every key present) and clustered (keys
    missing, so the pool is compacted); device and host id paths."""
    _say("upload_from_ids full size", kind)
    d_ids = bench.make_ids(torch) if kind == "uniform" else bench.clustered_ids(torch)[0]
    want, n_distinct = _bitset_of_ids(torch, d_ids)
    if kind == "uniform":
        assert n_distinct == bench.N_DISTINCT
    g = gpu.upload_from_device_ids(d_ids, U)
    assert torch.equal(_decoded(torch, gpu, g), want)
    _check_all_bitmap_ids_result(torch, gpu, g, want, n_distinct)
    gpu.free(g)
    _say("upload_from_ids full size host ids", kind)
    g = gpu.upload_from_ids(d_ids.cpu().numpy().view("uint32"), U)
    assert torch.equal(_decoded(torch, gpu, g), want)
    assert g.total_cardinality == n_distinct
    gpu.free(g)


def test_upload_from_ids_full_size_threshold_variants(gpu, torch):
    """BASELINE configs[1] names AUTO, KEEP_DEFAULT and ALL: above 1024 ids the
    reference builds all-bitmap whatever the threshold (src/upload_ids.cu:573-587),
    so the KEEP and ALL uploads of the 100M headline ids equal the AUTO one
    field by field, pools included."""
    from helpers import assert_same
    d_ids = bench.make_ids(torch)
    _say("upload_from_ids full size AUTO")
    g = gpu.upload_from_device_ids(d_ids, U)
    want = gpu.download(g)
    gpu.free(g)
    for name, thr in (("KEEP_DEFAULT", orc.PROMOTE_KEEP_DEFAULT), ("ALL", orc.PROMOTE_ALL)):
        _say("upload_from_ids full size", name)
        g = gpu.upload_from_device_ids(d_ids, U, thr)
        assert_same(gpu.download(g), want, strict=True, what=f"threshold {name}")
        gpu.free(g)


def test_upload_from_ids_full_size_complement(gpu, torch):
    """More than U/2 distinct ids: the complement is stored (negated) and
    decodes to the same set; total_cardinality is the logical count."""
    _say("upload_from_ids full size complement")
    i = torch.arange((U // 2) + (U // 8), device="cuda", dtype=torch.int64)
    d_ids = bench.bijective30(i, 3).to(torch.int32)
    want, n_distinct = _bitset_of_ids(torch, d_ids)
    g = gpu.upload_from_device_ids(d_ids, U)
    assert g.negated and g.total_cardinality == n_distinct
    assert torch.equal(_decoded(torch, gpu, g), want)
    gpu.free(g)


@pytest.mark.parametrize("density,seed", [(0.001, 20), (0.5, 21), (0.9, 22)])
def test_upload_from_device_bitset_full_size(gpu, torch, density, seed):
    """2^25 words: decode(upload(words)) == words; negated iff popcount > U/2."""
    _say("upload_from_device_bitset full size", density)
    w = bench._bitset_words(torch, density, seed)
    pc = int(_popcount_words(torch, w).sum().item())
    g = gpu.upload_from_device_bitset(w, U)
    assert g.negated == (pc > U // 2)
    assert g.total_cardinality == pc
    assert torch.equal(_decoded(torch, gpu, g), w)
    gpu.free(g)


OPS = {"and": (0, lambda a, b: a & b), "or": (1, lambda a, b: a | b),
       "andnot": (2, lambda a, b: a & ~b), "xor": (3, lambda a, b: a ^ b)}


@pytest.mark.parametrize("op", list(OPS))
def test_set_operation_full_size(gpu, torch, op):
    """Two 50% bitmaps over 2^30 (config 3, B x B'): decode(op(A, B)) ==
    op(words_A, words_B)."""
    _say("set_operation full size", op)
    code, f = OPS[op]
    wa = bench._bitset_words(torch, 0.5, 32)
    wb = bench._bitset_words(torch, 0.5, 33)
    a = gpu.upload_from_device_bitset(wa, U)
    b = gpu.upload_from_device_bitset(wb, U)
    r = gpu.set_operation(a, b, code)
    assert torch.equal(_decoded(torch, gpu, r), f(wa, wb))
    for x in (a, b, r):
        gpu.free(x)


def test_multi_and_full_size(gpu, torch):
    """k = 8 all-bitmap inputs over 2^30 (the fused path), densities
    {0.1, 1, 10, 50}% twice: decode == AND of the words."""
    _say("multi_and full size k=8")
    ws, gs = [], []
    for j, d in enumerate([0.001, 0.01, 0.1, 0.5] * 2):
        w = bench._bitset_words(torch, d, 40 + j)
        ws.append(w)
        gs.append(gpu.upload_from_device_bitset(w, U))
    r = gpu.multi_and(gs)
    want = ws[0]
    for w in ws[1:]:
        want = want & w
    assert torch.equal(_decoded(torch, gpu, r), want)
    for x in gs + [r]:
        gpu.free(x)


def test_contains_full_size(gpu, torch):
    """100M uniform queries against the headline bitmap, in the batched,
    wavefront and partitioned modes: the answer is the bit of the
    independently built bitset."""
    _say("contains full size")
    d_ids = bench.make_ids(torch)
    want, _ = _bitset_of_ids(torch, d_ids)
    g = gpu.upload_from_device_ids(d_ids, U)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(44)
    q = torch.randint(0, U, (100_000_000,), device="cuda", generator=gen, dtype=torch.int64)
    expect = ((want[q >> 5].to(torch.int64) >> (q & 31)) & 1).to(torch.int32)
    out = torch.empty(q.numel(), device="cuda", dtype=torch.int32)
    qi = q.to(torch.int32)
    del q
    for mode in (gpu.QUERY_CONTAINS, gpu.QUERY_WAVEFRONT, gpu.QUERY_PARTITIONED):
        out.fill_(7)
        gpu.contains_batch(g, qi, out, mode)
        torch.cuda.synchronize()
        assert torch.equal(out, expect), mode
    gpu.free(g)

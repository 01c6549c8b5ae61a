#!/usr/bin/env python3
"""Benchmark: upload_from_ids of 100M unsorted uint32 ids over U = 2^30 on one MI355X.

BASELINE.json configs[1] (the metric "upload ms @100M IDs"): 90M distinct
uniform ids plus 10M duplicates drawn from them, shuffled, already resident in
HBM; one step = one upload_from_device_ids() call (all kernels, its host
sync and the allocation of the result) plus the stream-ordered free.  Steps are
timed cold: a 512 MiB read evicts the 256 MB Infinity Cache before each step,
outside the step's interval.  The warm (back-to-back) figure is reported beside.

Also reported (extra fields, measured in the same run):
  roofline      the path's algorithmic bytes B = 4N + 8192 n_c + 9 n_c +
                2 (max_key + 1) over the path's device time: the sum of its
                kernels' mean launch times from HIP events recorded inside the
                library, on the library's stream, during the timed steps;
                `kernels` gives each kernel's own rate;
  cpu_baseline  the CPU port of the reference's upload (sort, unique, build) on
                a 10M-id sample, scaled x10, at 1 thread; `threads_n` is a
                threaded CPU build on the same sample at every host thread;
  secondary     BASELINE configs[0] on the CPU and the GPU; configs[2] (set
                operations over the A/B/C operands, multi_and fused and
                pairwise); configs[3] (point queries on both layouts at four
                densities); the fused filtered top-k; the other
                configs[1] variants; conversions, the portable format and the
                batch API -- each cold, with its CPU baseline where one applies.

--gpus N with N > 1 exits: this build measures one GPU only.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "cu-roaring-bitmap_amd", "python"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

HBM_PEAK_GBS = 8000.0
EVENT_EVERY = 4
U = 1 << 30
N_IDS = 100_000_000
N_DISTINCT = 90_000_000


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def bijective30(i, seed):
    """A permutation of [0, 2^30): xorshift-multiply rounds on 30-bit values (each step is invertible)."""
    import torch
    m = (1 << 30) - 1
    x = (i + seed) & m
    x = x ^ (x >> 15)
    x = (x * 0x2C1B3C6D) & m
    x = x ^ (x >> 13)
    x = (x * 0x297A2D39) & m
    x = x ^ (x >> 16)
    return x


def make_ids(torch, seed=10):
    dev = "cuda"
    i = torch.arange(N_DISTINCT, device=dev, dtype=torch.int64)
    distinct = bijective30(i, seed)
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 1)
    dup = distinct[torch.randint(0, N_DISTINCT, (N_IDS - N_DISTINCT,), device=dev, generator=g)]
    ids = torch.cat([distinct, dup])
    g.manual_seed(seed + 2)
    ids = ids[torch.randperm(N_IDS, device=dev, generator=g)]
    return ids.to(torch.int32).contiguous()


def upload_kernel_bytes(name, n, n_c, max_key):
    """Algorithmic bytes per launch of each upload kernel."""
    return {
        # read every id (4 B), write it back bucket-sorted within its tile as a 20-bit field (2.5 B)
        "ids_tile_sort": 4 * n + 5 * n // 2,
        # read the packed fields, write containers + per-key counts
        "ids_build": 5 * n // 2 + 8192 * n_c + 4 * n_c,
    }.get(name)


# The kernels of one device-resident upload_from_ids call on the headline input.
UPLOAD_PATH = ("ids_tile_sort", "ids_build", "ids_rank")


def evict(flush):
    """Read 512 MiB (twice the 256 MB Infinity Cache), leaving only clean lines of it cached."""
    import torch
    flush.view(torch.int64).sum()


def median(xs):
    xs = sorted(xs)
    return xs[len(xs) // 2]


def cold_time(torch, fn, iters, flush, after=None):
    """Median ms of fn() with the 256 MB Infinity Cache flushed before each call;
    after(result), if given, runs outside the timed interval (a result freed
    there returns its block to the library's cache, as in a steady state)."""
    ts = []
    for _ in range(iters):
        evict(flush)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        r = fn()
        torch.cuda.synchronize()
        ts.append((time.perf_counter() - t0) * 1e3)
        if after is not None:
            after(r)
    return median(ts)


def cold_time_and_kernels(torch, cr, fn, iters, flush, after=None):
    """cold_time() of fn with the library's kernel timer off (its event markers
    add queue time to every launch), then the per-kernel report of as many more
    cold calls with it on: the API time never carries the markers.  The report
    is {name: (launches, total_ms, median_ms)}; callers use the median."""
    t = cold_time(torch, fn, iters, flush, after=after)
    cr.timing_enable(True)
    cold_time(torch, fn, iters, flush, after=after)
    rep = cr.timing_report()
    cr.timing_enable(False)
    return t, rep


def kernel_medians(rep):
    """{kernel: median launch ms} from a timing report, host phases left out."""
    return {k: v[2] for k, v in rep.items() if not k.startswith("host:")}


# Lines whose summed kernel medians exceed the whole call's median time (the
# kernels of one call cannot take longer than the call): each is named here
# and counted in the headline line.
DEVICE_GT_API = []


def device_le_api(dev_ms, api_ms, tol=1.02):
    ok = bool(dev_ms <= api_ms * tol)
    if not ok:
        import inspect
        DEVICE_GT_API.append(f"{inspect.stack()[1].function}: device {dev_ms:.4f} ms > api {api_ms:.4f} ms")
        log("WARNING device time exceeds API time:", DEVICE_GT_API[-1])
    return ok


def cpu_median(fn, reps):
    """Median seconds (and the first answer) of `reps` runs of an orc CPU
    baseline call returning (seconds, answer, ...)."""
    runs = [fn() for _ in range(reps)]
    ts = sorted(r[0] for r in runs)
    return ts[len(ts) // 2], runs[0][1]


SECTIONS = ("config0", "config2", "config3", "conversions", "batch", "upload_variants", "promote_sweep", "topk")


def secondary(torch, cr, flush, no_cpu, sections):
    nt = cpu_threads()
    out = {"cpu": cpu_info()}
    if "config0" in sections:
        out["config0_2^24"] = config0(torch, cr, nt)
    if "config2" in sections:
        out["config2_set_ops_2^30"] = config2(torch, cr, flush, nt, no_cpu)
        torch.cuda.empty_cache()
    if "config3" in sections:
        out["config3_point_queries_2^30"] = config3(torch, cr, flush, nt, no_cpu)
    if "conversions" in sections:
        conversion_sections(torch, cr, flush, out)
    if "batch" in sections:
        out["batch_16x2^28"] = batch_api(torch, cr, flush)
        torch.cuda.empty_cache()
    if "upload_variants" in sections:
        out["upload_variants_2^30"] = upload_variants(torch, cr)
    if "promote_sweep" in sections:
        out["promote_auto_sweep"] = promote_sweep(torch, cr, flush)
    return out


def conversion_sections(torch, cr, flush, out):
    """The conversions and the portable format on a 10% all-bitmap 2^30 bitmap
    and a 0.5% array-container one."""
    ids = bijective30(torch.arange(int(0.1 * U), device="cuda", dtype=torch.int64), 40).to(torch.int32)
    bm = cr.upload_from_device_ids(ids, U)
    del ids
    torch.cuda.empty_cache()
    sparse = sparse_arrays(cr, 0.005, 60)
    out["conversions_2^30"] = conversions(torch, cr, flush, {"dense_10pct_bitmap": bm, "sparse_0.5pct_array": sparse})
    out["portable_format_2^30"] = portable(torch, cr, flush, {"dense_10pct_bitmap": bm, "sparse_0.5pct_array": sparse})
    cr.free(sparse)
    cr.free(bm)
    torch.cuda.empty_cache()


# ---- BASELINE configs[0], [2], [3]: operands, timings and CPU baselines ------------
def cpu_threads():
    """Host threads for the threaded CPU baselines: every hardware thread of the
    process's CPU share, at most 16 (the GPU box's share per GPU)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return max(1, min(16, n))


def cpu_info():
    """The host CPU as /proc/cpuinfo and lscpu describe it (a virtualised box
    may report only "AMD EPYC" as its model name, so family/model/stepping,
    cache and vector-ISA flags are kept too)."""
    info = {"model": "unknown"}
    keys = {"model name": "model", "cpu family": "family", "model": "model_number", "stepping": "stepping",
            "cache size": "cache"}
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k = k.strip()
            if k in keys and keys[k] not in info or (k == "model name" and info["model"] == "unknown"):
                info[keys[k]] = v.strip()
            if k == "flags":
                fl = set(v.split())
                info["isa"] = [f for f in ("avx2", "avx512f", "avx512_bf16", "avx512_vnni") if f in fl]
            if not line.strip() and "family" in info:
                break
    except OSError:
        pass
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        want = ("Model name", "Socket(s)", "Core(s) per socket", "Thread(s) per core", "L3 cache", "CPU max MHz")
        info["lscpu"] = {k: v.strip() for k, _, v in (ln.partition(":") for ln in out.splitlines()) if k.strip() in want}
    except Exception:
        pass
    info.update({"os_cpu_count": os.cpu_count(), "threads_used": cpu_threads()})
    return info


def words_bernoulli(torch, density, seed, universe=U):
    """A flat bitset (host u64 words) of `universe` ids at `density`: exact
    Bernoulli(1/2) per bit at 50%, else density * U uniform draws (duplicates
    merge), on the device."""
    import numpy as np
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    nw = universe // 32
    if density == 0.5:
        w = torch.randint(-(1 << 31), 1 << 31, (nw,), device="cuda", generator=g, dtype=torch.int64).to(torch.int32)
    else:
        ids = torch.unique(torch.randint(0, universe, (int(density * universe),), device="cuda", generator=g))
        w64 = torch.zeros(nw, device="cuda", dtype=torch.int64)
        w64.index_add_(0, ids >> 5, torch.ones_like(ids) << (ids & 31))  # distinct bits: the sum is the OR
        w = (w64 - (w64 >= (1 << 31)).to(torch.int64) * (1 << 32)).to(torch.int32)
        del ids, w64
    return np.ascontiguousarray(w.cpu().numpy()).view(np.uint64)


def words_runs(coverage, seed, universe=U):
    """Runs of length U[1000, 65536) at uniform starts until they cover
    `coverage` of the universe (overlaps merge), as host u64 words."""
    import numpy as np
    rng = np.random.default_rng(seed)
    nw = universe // 64
    w = np.zeros(nw, dtype=np.uint64)
    covered, target = 0, int(coverage * universe)
    full = np.uint64(0xFFFFFFFFFFFFFFFF)
    while covered < target:
        ln = int(rng.integers(1000, 65536))
        st = int(rng.integers(0, universe - ln))
        e = st + ln
        a, b = st >> 6, (e - 1) >> 6
        lo_mask = full << np.uint64(st & 63)
        hi_mask = full >> np.uint64(63 - ((e - 1) & 63))
        if a == b:
            w[a] |= lo_mask & hi_mask
        else:
            w[a] |= lo_mask
            w[a + 1:b] = full
            w[b] |= hi_mask
        covered += ln
    return w


def keep_upload(cr, lite, universe=U):
    """The packed upload with PROMOTE_KEEP_DEFAULT (container types kept), not
    negated (universe inferred from the last key, no complement)."""
    return cr.upload_containers(lite.containers(), 0, False, 0, cr.PROMOTE_KEEP_DEFAULT)


def container_bytes(cr, g):
    """Host (keys, per-container payload bytes): bitmap 8192, array 2 card, run 4 n_runs."""
    import numpy as np
    n = g.n_containers
    keys = cr._d2h(g.keys, n, np.uint16)
    types = cr._d2h(g.types, n, np.uint8)
    cards = cr._d2h(g.cardinalities, n, np.uint16).astype(np.int64)
    b = np.where(types == 1, 8192, np.where(types == 0, 2 * cards, 4 * cards))
    return keys, b


def setop_algorithmic_bytes(cr, a, b, r, op):
    """Input containers that take part in `op`, the output containers, 9 B of
    metadata per container in and out."""
    import numpy as np
    ka, ba = container_bytes(cr, a)
    kb, bb = container_bytes(cr, b)
    ia = np.isin(ka, kb)
    ib = np.isin(kb, ka)
    if op == cr.AND:
        nin, byin = ia.sum() + ib.sum(), ba[ia].sum() + bb[ib].sum()
    elif op == cr.ANDNOT:
        nin, byin = ka.size + ib.sum(), ba.sum() + bb[ib].sum()
    else:
        nin, byin = ka.size + kb.size, ba.sum() + bb.sum()
    out = 8192 * r.n_bitmap_containers + r.array_pool_bytes + r.run_pool_bytes
    return int(byin + out + 9 * (nin + r.n_containers))


def config0(torch, cr, nt):
    """BASELINE configs[0] at U = 2^24: A 1% and B 10% uniform draws (with
    replacement), AND/OR/ANDNOT/XOR with their cardinalities, then 1M uniform
    point queries.  CPU: roaring-lite at 1 thread (CRoaring's algorithms).
    GPU: the same work through the library (ids already on the device), warm."""
    import numpy as np
    import orc
    U0 = 1 << 24
    rng1, rng2, rng3 = (np.random.default_rng(s) for s in (1, 2, 3))
    a = rng1.integers(0, U0, 167_772, dtype=np.uint64).astype(np.uint32)
    b = rng2.integers(0, U0, 1_677_722, dtype=np.uint64).astype(np.uint32)
    q = rng3.integers(0, U0, 1_000_000, dtype=np.uint64).astype(np.uint32)
    ts = [orc.cpu_config0(a, b, q) for _ in range(3)]
    t_cpu, parts, cards, hits = sorted(ts, key=lambda x: x[0])[1]
    da = torch.from_numpy(a.view(np.int32)).cuda()
    db = torch.from_numpy(b.view(np.int32)).cuda()
    dq = torch.from_numpy(q.view(np.int32)).cuda()
    res = torch.empty_like(dq)

    def gpu_run():
        ga = cr.upload_from_device_ids(da, U0)
        gb = cr.upload_from_device_ids(db, U0)
        t1 = time.perf_counter()
        c = []
        for op in (cr.AND, cr.OR, cr.ANDNOT, cr.XOR):
            r = cr.set_operation(ga, gb, op)
            c.append(cr.cardinality(r))
            cr.free_async(r)
        t2 = time.perf_counter()
        cr.contains_batch(ga, dq, res, cr.QUERY_CONTAINS)
        torch.cuda.synchronize()
        t3 = time.perf_counter()
        cr.free_async(ga)
        cr.free_async(gb)
        return c, (t1, t2, t3)
    gpu_run()
    torch.cuda.synchronize()
    runs = []
    for _ in range(5):
        t0 = time.perf_counter()
        c, (t1, t2, t3) = gpu_run()
        torch.cuda.synchronize()
        runs.append(((time.perf_counter() - t0) * 1e3, (t1 - t0) * 1e3, (t2 - t1) * 1e3, (t3 - t2) * 1e3, c))
    runs.sort(key=lambda x: x[0])
    g_ms, g_build, g_ops, g_q, g_cards = runs[len(runs) // 2]
    g_hits = int(res.sum().item())
    assert g_cards == cards and g_hits == hits, ("configs[0] GPU and CPU disagree", g_cards, cards, g_hits, hits)
    out = {"universe": U0, "a_draws": int(a.size), "b_draws": int(b.size), "queries": int(q.size),
           "cardinalities_and_or_andnot_xor": cards, "query_hits": hits,
           "cpu_1t": {"ms": round(t_cpu * 1e3, 3), "build_ms": round(parts[0] * 1e3, 3),
                      "ops_ms": round(parts[1] * 1e3, 3), "queries_ms": round(parts[2] * 1e3, 3),
                      "Mqps": round(q.size / parts[2] / 1e6, 2)},
           "gpu": {"ms": round(g_ms, 3), "build_ms": round(g_build, 3), "ops_with_cardinality_ms": round(g_ops, 3),
                   "queries_ms": round(g_q, 3), "note": "warm; ids on the device; each call synchronises"},
           "same_answers": True}
    log("configs[0]", out["cpu_1t"]["ms"], "ms CPU,", out["gpu"]["ms"], "ms GPU")
    return out


def config2_operands(torch, cr):
    """configs[2] over 2^30: A/A' 0.1% (array containers), B/B' 50% (bitmaps),
    C/C' runs U[1k,64k) to 20% (run_optimize -> run containers), as roaring-lite
    bitmaps and their KEEP uploads.  Returns {name: (Lite, GpuRoaring)}."""
    import orc
    ops = {}
    for name, make in (("A", lambda: words_bernoulli(torch, 0.001, 30)), ("A'", lambda: words_bernoulli(torch, 0.001, 31)),
                       ("B", lambda: words_bernoulli(torch, 0.5, 32)), ("B'", lambda: words_bernoulli(torch, 0.5, 33)),
                       ("C", lambda: words_runs(0.2, 34)), ("C'", lambda: words_runs(0.2, 35))):
        lite = orc.Lite.from_words(make())
        if name.startswith("C"):
            lite.run_optimize()
        ops[name] = (lite, keep_upload(cr, lite))
    return ops


SETOP_PAIRS = (("A", "B"), ("B", "A"), ("A", "C"), ("C", "A"), ("B", "C"), ("C", "B"),
               ("A", "A'"), ("B", "B'"), ("C", "C'"))


def config2(torch, cr, flush, nt, no_cpu):
    """the nine operand pairs x four operations (cold, median of 3),
    GB/s of the algorithmic bytes; the CPU baseline at 1 and nt threads."""
    import orc
    ops = config2_operands(torch, cr)
    names = {cr.AND: "AND", cr.OR: "OR", cr.ANDNOT: "ANDNOT", cr.XOR: "XOR"}
    out = {"operands": {k: {"containers": v[1].n_containers, "bitmap": v[1].n_bitmap_containers,
                            "array": v[1].n_array_containers, "run": v[1].n_run_containers,
                            "cardinality": int(v[0].cardinality())} for k, v in ops.items()}}
    shards = {} if no_cpu else {k: v[0].shards(4 * nt, U >> 16) for k, v in ops.items()}
    for x, y in SETOP_PAIRS:
        (la, ga), (lb, gb) = ops[x], ops[y]
        for op, oname in names.items():
            r = cr.set_operation(ga, gb, op)  # untimed first call
            nbytes = setop_algorithmic_bytes(cr, ga, gb, r, op)
            card = cr.cardinality(r)
            cr.free(r)
            t, rep = cold_time_and_kernels(torch, cr, lambda: cr.set_operation(ga, gb, op), 3, flush, after=cr.free)
            kern = kernel_medians(rep)
            dev = sum(kern.values())
            exec_ms = kern.get("so_exec_bb", kern.get("so_exec", float("nan")))
            line = {"algorithmic_bytes": nbytes, "api_ms": round(t, 4), "api_GBps": round(nbytes / t / 1e6, 1),
                    "device_ms": round(dev, 4), "device_GBps": round(nbytes / dev / 1e6, 1),
                    "exec_kernel_ms": round(exec_ms, 4),
                    "exec_frac_of_hbm_peak": round(nbytes / exec_ms / 1e6 / HBM_PEAK_GBS, 4),
                    "cardinality": card, "kernels_ms": {k: round(v, 4) for k, v in kern.items()},
                    "device_le_api": device_le_api(dev, t)}
            if not no_cpu:
                t1, c1 = cpu_median(lambda: orc.cpu_setop([la], [lb], op, 1), 3)
                tn, cn = cpu_median(lambda: orc.cpu_setop(shards[x], shards[y], op, nt), 7)
                # The reference stores a full (65536) result container's card as 0
                # and then drops zero-card results of AND/ANDNOT/XOR
                # (src/set_ops.cu:179-180,1111,1145); roaring-lite keeps them.
                dropped = c1 - card
                assert c1 == cn and dropped >= 0 and dropped % 65536 == 0 and (op != cr.OR or dropped == 0), \
                    (x, y, oname, c1, cn, card)
                line["cpu_1t_ms"] = round(t1 * 1e3, 3)
                line[f"cpu_{nt}t_ms"] = round(tn * 1e3, 3)
                if dropped:
                    line["full_containers_dropped_as_in_reference"] = dropped // 65536
            out[f"{x}{y}_{oname}"] = line
        log("set ops", x, y, {o: out[f"{x}{y}_{o}"]["api_ms"] for o in names.values()})
    # multi_and from KEEP uploads of Bernoulli bitmaps: pairwise (mixed types), and
    # the fused path on all-bitmap uploads of the same sets
    for k, dens in ((3, (0.001, 0.1, 0.5)), (8, (0.001, 0.001, 0.01, 0.01, 0.1, 0.1, 0.5, 0.5))):
        lites = [orc.Lite.from_words(words_bernoulli(torch, d, 100 + i)) for i, d in enumerate(dens)]
        for route, mk in (("pairwise_keep", lambda lt: keep_upload(cr, lt)),
                          ("fused_all_bitmap", lambda lt: cr.upload_containers(lt.containers(), 0, False, 0,
                                                                               cr.PROMOTE_ALL))):
            ins = [mk(lt) for lt in lites]
            r = cr.multi_and(ins)
            card = cr.cardinality(r)
            n_common = r.n_containers
            outb = 8192 * r.n_bitmap_containers + r.array_pool_bytes + r.run_pool_bytes
            cr.free(r)
            t, rep = cold_time_and_kernels(torch, cr, lambda: cr.multi_and(ins), 3, flush, after=cr.free)
            inb = sum(int(container_bytes(cr, g)[1].sum()) + 9 * g.n_containers for g in ins)
            kern = kernel_medians(rep)
            line = {"densities": list(dens), "route": route, "n_result_containers": n_common, "cardinality": card,
                    "api_ms": round(t, 4), "device_ms": round(sum(kern.values()), 4),
                    "kernels_ms": {kk: round(v, 4) for kk, v in kern.items()},
                    "device_le_api": device_le_api(sum(kern.values()), t)}
            if route == "fused_all_bitmap":
                mb = (k + 1) * 8192 * n_common + 9 * (k + 1) * n_common
                ka = kern.get("mand_and", float("nan"))
                line.update({"algorithmic_bytes": mb, "mand_and_GBps": round(mb / ka / 1e6, 1),
                             "mand_and_frac_of_hbm_peak": round(mb / ka / 1e6 / HBM_PEAK_GBS, 4),
                             "api_GBps": round(mb / t / 1e6, 1)})
            else:
                line.update({"input_bytes": inb, "output_bytes": outb})
            for g in ins:
                cr.free(g)
            out[f"multi_and_k{k}_{route}"] = line
        if not no_cpu:
            t1, c1 = cpu_median(lambda: orc.cpu_multi_and([[lt] for lt in lites], 1), 3)
            shl = [lt.shards(4 * nt, U >> 16) for lt in lites]
            tn, cn = cpu_median(lambda: orc.cpu_multi_and(shl, nt), 7)
            assert c1 == cn == out[f"multi_and_k{k}_fused_all_bitmap"]["cardinality"] == \
                out[f"multi_and_k{k}_pairwise_keep"]["cardinality"]
            out[f"multi_and_k{k}_cpu"] = {"cpu_1t_ms": round(t1 * 1e3, 3), f"cpu_{nt}t_ms": round(tn * 1e3, 3),
                                          "algorithm": "copy of the first input ANDed with each other one"}
        log(f"multi_and k={k}", {r_: out[f"multi_and_k{k}_{r_}"]["api_ms"] for r_ in ("pairwise_keep",
                                                                                    "fused_all_bitmap")})
    for _, g in ops.values():
        cr.free(g)
    return out


def query_sets(torch, nq=100_000_000):
    """configs[3] queries: uniform over 2^30 (seed 44), and sorted-clustered
    (each group of 4096 uniform within one random 65536-aligned window, sorted;
    seed 45)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(44)
    q_uni = torch.randint(0, U, (nq,), device="cuda", generator=g, dtype=torch.int64).to(torch.int32)
    g.manual_seed(45)
    win = torch.randint(0, U >> 16, (nq // 4096,), device="cuda", generator=g, dtype=torch.int64)
    off = torch.randint(0, 65536, (nq // 4096, 4096), device="cuda", generator=g, dtype=torch.int64)
    q_clu = ((win[:, None] << 16) + off.sort(dim=1).values).reshape(-1).to(torch.int32)
    return {"uniform": q_uni, "clustered": q_clu}


def config3(torch, cr, flush, nt, no_cpu):
    """Bernoulli bitmaps over 2^30 at 0.1/1/10/50% (seeds 40-43) in
    the compressed layout (KEEP upload: arrays at 0.1/1%) and the promoted one
    (ALL), 100M uniform and sorted-clustered queries, every query mode, cold.
    Gq/s and the fraction of HBM peak at 18 B per query.  CPU: roaring-lite
    contains on a 10M-query uniform sample at 1 and nt threads."""
    import numpy as np
    import orc
    qs = query_sets(torch)
    nq = qs["uniform"].numel()
    res = torch.empty(nq, device="cuda", dtype=torch.int32)
    modes = {"contains": cr.QUERY_CONTAINS, "wavefront_contains": cr.QUERY_WAVEFRONT,
             "wavefront_contains_api": cr.QUERY_WAVEFRONT_API, "contains_api": cr.QUERY_CONTAINS_API,
             "partitioned": cr.QUERY_PARTITIONED}
    out = {"queries": nq}
    for j, dens in enumerate((0.001, 0.01, 0.1, 0.5)):
        lite = orc.Lite.from_words(words_bernoulli(torch, dens, 40 + j))
        layouts = {"compressed": keep_upload(cr, lite),
                   "promoted": cr.upload_containers(lite.containers(), 0, False, 0, cr.PROMOTE_ALL)}
        d = {"cardinality": int(lite.cardinality()),
             "compressed_types": {"array": layouts["compressed"].n_array_containers,
                                  "bitmap": layouts["compressed"].n_bitmap_containers}}
        ref = None
        for lname, g in layouts.items():
            for qname, q in qs.items():
                for mname, mode in modes.items():
                    cr.contains_batch(g, q, res, mode)
                    torch.cuda.synchronize()
                    t = cold_time(torch, lambda: cr.contains_batch(g, q, res, mode), 3, flush)
                    d[f"{lname}_{qname}_{mname}_Gqps"] = round(nq / t / 1e6, 2)
                    if mname in ("contains", "partitioned"):
                        d[f"{lname}_{qname}_{mname}_frac_hbm_18B"] = round(18 * nq / t / 1e6 / HBM_PEAK_GBS, 4)
                    # every mode and layout gives the same answers (checksum of the answer vector)
                    s_ = int((res.to(torch.int64) * (torch.arange(nq, device="cuda") % 1021 + 1)).sum().item())
                    key = qname
                    if ref is None:
                        ref = {}
                    if key not in ref:
                        ref[key] = s_
                    assert ref[key] == s_, ("query modes disagree", dens, lname, qname, mname)
        if not no_cpu:
            hq = qs["uniform"][:10_000_000].cpu().numpy().view(np.uint32)
            t1, a1 = orc.cpu_contains(lite, hq[:2_000_000], 1)
            tn, an = orc.cpu_contains(lite, hq, nt)
            d["cpu_1t_Mqps"] = round(2_000_000 / t1 / 1e6, 2)
            d[f"cpu_{nt}t_Mqps"] = round(hq.size / tn / 1e6, 2)
            # the CPU answers equal the GPU's on the sample
            cr.contains_batch(layouts["compressed"], qs["uniform"][:10_000_000], res[:10_000_000], cr.QUERY_CONTAINS)
            torch.cuda.synchronize()
            assert np.array_equal(an, res[:10_000_000].cpu().numpy().view(np.uint32)), "CPU and GPU answers differ"
        for g in layouts.values():
            cr.free(g)
        out[f"density_{dens * 100:g}pct"] = d
        log("configs[3]", dens, {k: v for k, v in d.items() if k.endswith("contains_Gqps") or "partitioned_Gqps" in k})
    del qs, res
    torch.cuda.empty_cache()
    return out


def promote_sweep(torch, cr, flush):
    """PROMOTE_AUTO on gfx950, from measurement: the compressed layout (KEEP:
    arrays up to 4096 values) against the promoted one (ALL: every container
    an 8 KiB bitmap) over U = 2^20 .. 2^30 at 0.1 / 1 / 10% density.  For each:
    10M uniform and 10M sorted-clustered point queries (Gq/s, cold) and the AND
    of two such bitmaps (API ms, cold), plus each layout's bytes.  The ratio
    promoted / compressed > 1 means promotion pays."""
    import orc
    res = {}
    nq = 10_000_000
    out = torch.empty(nq, device="cuda", dtype=torch.int32)
    for lg in (20, 22, 24, 26, 28, 30):
        Uu = 1 << lg
        g = torch.Generator(device="cuda")
        g.manual_seed(900 + lg)
        q_uni = torch.randint(0, Uu, (nq,), device="cuda", generator=g, dtype=torch.int64).to(torch.int32)
        nwin = max(1, Uu >> 16)
        win = torch.randint(0, nwin, (nq // 4096,), device="cuda", generator=g, dtype=torch.int64)
        off = torch.randint(0, min(65536, Uu), (nq // 4096, 4096), device="cuda", generator=g, dtype=torch.int64)
        q_clu = ((win[:, None] << 16) + off.sort(dim=1).values).reshape(-1).to(torch.int32)
        for dens in (0.001, 0.01, 0.1):
            lites = [orc.Lite.from_words(words_bernoulli(torch, dens, 910 + lg + i, universe=Uu)) for i in (0, 1)]
            row = {}
            for lname, thr in (("compressed", cr.PROMOTE_KEEP_DEFAULT), ("promoted", cr.PROMOTE_ALL)):
                gs = [cr.upload_containers(lt.containers(), Uu, False, lt.cardinality(), thr) for lt in lites]
                a = gs[0]
                row[f"{lname}_bytes"] = int(8192 * a.n_bitmap_containers + a.array_pool_bytes + a.run_pool_bytes +
                                            9 * a.n_containers + 2 * (a.max_key + 1))
                for qname, q in (("uniform", q_uni), ("clustered", q_clu)):
                    cr.contains_batch(a, q, out, cr.QUERY_CONTAINS)
                    t = cold_time(torch, lambda: cr.contains_batch(a, q, out, cr.QUERY_CONTAINS), 3, flush)
                    row[f"{lname}_{qname}_Gqps"] = round(nq / t / 1e6, 2)
                cr.free(cr.set_operation(gs[0], gs[1], cr.AND))
                row[f"{lname}_and_ms"] = round(cold_time(torch, lambda: cr.set_operation(gs[0], gs[1], cr.AND), 3,
                                                         flush, after=cr.free), 4)
                for x in gs:
                    cr.free(x)
            for k in ("uniform_Gqps", "clustered_Gqps"):
                row[f"promoted_over_compressed_{k}"] = round(row[f"promoted_{k}"] / row[f"compressed_{k}"], 3)
            row["promoted_over_compressed_and_speed"] = round(row["compressed_and_ms"] / row["promoted_and_ms"], 3)
            res[f"2^{lg}_{dens * 100:g}pct"] = row
            log("promote sweep", lg, dens, {k: v for k, v in row.items() if "over" in k})
        del q_uni, q_clu, win, off
    res["device_l2_bytes"] = cr.device_l2_bytes()
    res["auto_threshold"] = {f"2^{lg}": cr.resolve_auto_threshold(1 << lg) for lg in (20, 22, 24, 26, 28, 30)}
    return res


def clustered_ids(torch, seed=11):
    """BASELINE configs[1], clustered variant: runs of length U[1000, 65536) at
    uniform starts over 2^30 until 90M ids (overlapping runs add duplicates),
    plus 10M duplicates drawn from them, shuffled."""
    dev = "cuda"
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    lens = torch.randint(1000, 65536, (2 * N_DISTINCT // 33268 + 64,), device=dev, generator=g)
    csum = torch.cumsum(lens, 0)
    n_runs = int(torch.searchsorted(csum, torch.tensor([N_DISTINCT], device=dev)).item()) + 1
    lens = lens[:n_runs].clone()
    lens[-1] -= int(csum[n_runs - 1].item()) - N_DISTINCT
    starts = torch.randint(0, U - 65536, (n_runs,), device=dev, generator=g)
    offs = torch.cumsum(lens, 0) - lens
    run_of = torch.repeat_interleave(torch.arange(n_runs, device=dev), lens)
    ids = starts[run_of] + (torch.arange(N_DISTINCT, device=dev) - offs[run_of])
    del run_of
    dup = ids[torch.randint(0, N_DISTINCT, (N_IDS - N_DISTINCT,), device=dev, generator=g)]
    ids = torch.cat([ids, dup])
    ids = ids[torch.randperm(N_IDS, device=dev, generator=g)]
    return ids.to(torch.int32).contiguous(), n_runs


def _bitset_words(torch, density, seed):
    """2^25 u32 words (a 2^30-bit bitset, as int32) at the given density."""
    dev = "cuda"
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    nw = U // 32
    if density == 0.5:
        return torch.randint(-(1 << 31), 1 << 31, (nw,), device=dev, generator=g, dtype=torch.int64).to(torch.int32)
    p = density if density < 0.5 else 1.0 - density
    ids = torch.unique(torch.randint(0, U, (int(p * U),), device=dev, generator=g))
    w = torch.zeros(nw, device=dev, dtype=torch.int64)
    w.index_add_(0, ids >> 5, torch.ones_like(ids) << (ids & 31))  # distinct bits: the sum is the OR
    del ids
    w = (w - (w >= (1 << 31)).to(torch.int64) * (1 << 32)).to(torch.int32)
    return w if density < 0.5 else torch.bitwise_not(w)


def upload_variants(torch, cr):
    """The rest of BASELINE configs[1]: upload_from_ids on the clustered
    variant (most keys absent, so the result is compacted), and
    upload_from_device_bitset at 0.1%, 50% and 90% density (the last one
    stored as the complement).  Hot timings (median of 5) with the kernels'
    HIP-event times; the bitset path's algorithmic bytes are the bitset read
    twice (count, compact) plus the containers written."""
    res = {}
    d, n_runs = clustered_ids(torch)
    torch.cuda.synchronize()

    def timed(fn):
        # Results are freed stream-ordered, as in the headline loop, so each
        # call's allocations come from the stream's pool.
        r = fn()
        torch.cuda.synchronize()
        meta = (r.n_containers, r.total_cardinality, bool(r.negated))
        cr.free_async(r)

        def calls():
            ts = []
            for _ in range(5):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                r = fn()
                torch.cuda.synchronize()
                ts.append((time.perf_counter() - t0) * 1e3)
                cr.free_async(r)
            return median(ts)
        t = calls()  # the kernel timer off: its markers would add queue time
        cr.timing_enable(True)
        calls()
        rep = cr.timing_report()
        cr.timing_enable(False)
        return t, meta, {k: round(v[2], 4) for k, v in rep.items()}

    t, (nc, card, neg), k = timed(lambda: cr.upload_from_device_ids(d, U))
    res["ids_clustered_100M"] = {"ms": round(t, 4), "runs": n_runs, "containers": nc, "distinct": card,
                                 "kernels_ms": k}
    del d
    torch.cuda.empty_cache()
    # Sparse uploads at 2^30: up to 1024 ids take the small path; above that,
    # fewer ids than keys (16384) build each container at its rank in a pool of
    # n slots; from 16384 ids on the pool is addressed by key.
    g = torch.Generator(device="cuda")
    g.manual_seed(74)
    for n_s in (1000, 1025, 10_000, 100_000, 1_000_000):
        ids_s = torch.randint(0, U, (n_s,), device="cuda", generator=g, dtype=torch.int64).to(torch.int32)
        t, (nc, card, neg), k = timed(lambda: cr.upload_from_device_ids(ids_s, U))
        res[f"ids_sparse_{n_s}"] = {"ms": round(t, 4), "containers": nc, "distinct": card, "kernels_ms": k}
    log("sparse uploads", {kk: v["ms"] for kk, v in res.items() if kk.startswith("ids_sparse")})
    for dens, seed in ((0.001, 71), (0.5, 72), (0.9, 73)):
        w = _bitset_words(torch, dens, seed)
        torch.cuda.synchronize()
        t, (nc, card, neg), k = timed(lambda: cr.upload_from_device_bitset(w, U))
        nbytes = 2 * (U // 8) + 8192 * nc + 9 * nc
        dev_ms = sum(v for kk, v in k.items() if not kk.startswith("host:"))
        res[f"bitset_{dens * 100:g}pct"] = {"ms": round(t, 4), "containers": nc, "cardinality": card,
                                            "negated": neg, "algorithmic_bytes": nbytes,
                                            "device_ms": round(dev_ms, 4),
                                            "device_GBps": round(nbytes / dev_ms / 1e6, 1),
                                            "frac_of_hbm_peak": round(nbytes / dev_ms / 1e6 / HBM_PEAK_GBS, 4),
                                            "kernels_ms": k}
        del w
        torch.cuda.empty_cache()
    log("upload variants", res)
    return res


def _kernel_line(rep, name, nbytes, t_api):
    k = rep.get(name, (1, float("nan"), float("nan")))[2]
    return {"algorithmic_bytes": nbytes, "api_ms": round(t_api, 4), f"{name}_ms": round(k, 4),
            f"{name}_GBps": round(nbytes / k / 1e6, 1), "frac_of_hbm_peak": round(nbytes / k / 1e6 / HBM_PEAK_GBS, 4),
            "kernels_ms": {kk: round(v, 4) for kk, v in kernel_medians(rep).items()},
            "device_le_api": device_le_api(sum(kernel_medians(rep).values()), t_api)}


def portable(torch, cr, flush, bitmaps):
    """Roaring portable-format serialize (device planning + payload kernels, then
    the copy of the bytes to host memory) and deserialize (host header parse,
    then the packed upload).  Kernel bytes: ps_plan reads the payloads and
    metadata; ps_write reads them again and writes the serialized payloads."""
    res = {}
    for name, g in bitmaps.items():
        import ctypes as C
        import numpy as np
        payload = 8192 * g.n_bitmap_containers + g.array_pool_bytes + g.run_pool_bytes + 9 * g.n_containers
        data = cr.portable_serialize(g)
        # the C calls are timed on pre-touched numpy buffers (no Python marshalling)
        hbuf = np.ones(len(data), dtype=np.uint8)
        w = C.c_size_t()
        lib = cr.load()

        def ser():
            assert lib.cr_portable_serialize(C.byref(g), None, hbuf.ctypes.data, hbuf.size, C.byref(w)) == 0
        t_ser, rep = cold_time_and_kernels(torch, cr, ser, 3, flush)
        assert hbuf.tobytes() == data
        kw = rep.get("ps_write", (1, float("nan"), float("nan")))[2]
        kp = rep.get("ps_plan", (1, float("nan"), float("nan")))[2]
        write_bytes = payload + len(data)
        r = {"serialized_bytes": len(data), "serialize_api_ms": round(t_ser, 3),
             "serialize_api_GBps_of_output": round(len(data) / t_ser / 1e6, 2),
             "ps_plan_ms": round(kp, 4), "ps_plan_GBps": round(payload / kp / 1e6, 1),
             "ps_write_ms": round(kw, 4), "ps_write_GBps": round(write_bytes / kw / 1e6, 1),
             "kernels_ms": {k: round(v, 4) for k, v in kernel_medians(rep).items()},
             "device_le_api": device_le_api(sum(kernel_medians(rep).values()), t_ser)}
        h = cr.GpuRoaring()
        ts = []
        for _ in range(4):
            t0 = time.perf_counter()
            assert lib.cr_portable_deserialize(hbuf.ctypes.data, hbuf.size, U, None, cr.PROMOTE_KEEP_DEFAULT,
                                               C.byref(h)) == 0
            ts.append((time.perf_counter() - t0) * 1e3)
            cr.free(h)
        ts = ts[1:]
        r["deserialize_api_ms"] = round(median(ts), 3)
        r["deserialize_api_GBps_of_input"] = round(len(data) / median(ts) / 1e6, 2)
        r["note"] = "API times include the PCIe copy of the serialized bytes (device to host, or host to device)"
        res[name] = r
        log("portable", name, r["serialize_api_ms"], "ms serialize", r["deserialize_api_ms"], "ms deserialize")
    return res


def batch_api(torch, cr, flush):
    """The batch API on 16 bitmaps over 2^28 (4096 keys each): eight 50%-dense
    (bitset containers) and eight 1% (array containers).  upload_batch from host
    containers; promote_batch; multi_and over the eight dense bitmaps and over
    four dense + four sparse (promoted); decompress_batch of all 16; 100M
    contains with a random bitmap per query, and through one view."""
    import numpy as np
    Ub = 1 << 28
    nk = Ub >> 16
    rng = np.random.default_rng(70)
    lists = []
    for b in range(16):
        if b < 8:
            words = rng.integers(0, np.iinfo(np.uint64).max, size=(nk, 1024), dtype=np.uint64, endpoint=True)
            cards = np.bitwise_count(words).sum(axis=1, dtype=np.int64)
            lists.append([(k, cr.TC_BITSET, int(cards[k]), words[k]) for k in range(nk)])
        else:
            ids = np.unique(rng.integers(0, Ub, int(0.01 * Ub), dtype=np.uint64))
            bounds = np.searchsorted(ids, np.arange(nk + 1, dtype=np.uint64) << np.uint64(16))
            lists.append([(k, cr.TC_ARRAY, int(bounds[k + 1] - bounds[k]),
                           (ids[bounds[k]:bounds[k + 1]] & np.uint64(0xFFFF)).astype(np.uint16))
                          for k in range(nk) if bounds[k + 1] > bounds[k]])
    # the container descriptors are marshalled once, outside the timed call
    import ctypes as C
    arrays = [cr._container_array(c) for c in lists]
    ptrs = (C.c_void_p * 16)(*[C.addressof(a[0]) for a in arrays])
    counts = (C.c_uint32 * 16)(*[len(c) for c in lists])
    B = cr.RoaringBatch()
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        rc = cr.load().cr_upload_batch(ptrs, counts, 16, None, C.byref(B))
        ts.append((time.perf_counter() - t0) * 1e3)
        assert rc == 0, cr.load().cr_last_error()
        if len(ts) < 3:
            cr.free_batch(B)
    t_up = median(ts)
    del arrays
    up_bytes = 8 * 8192 * nk + B.array_pool_bytes + 9 * B.total_containers
    del lists
    res = {"bitmaps": 16, "universe": Ub, "containers": B.total_containers,
           "upload_batch": {"api_ms": round(t_up, 2), "bytes": up_bytes, "GBps": round(up_bytes / t_up / 1e6, 2),
                            "note": "host containers packed into pinned memory, one host-to-device copy"}}
    T = B.total_containers
    # results are freed outside the timed intervals (allocations then come from
    # the library's cache, as in a steady state)
    P = cr.promote_batch(B)  # also the first launch (code object load), out of the timing
    torch.cuda.synchronize()
    t, rep = cold_time_and_kernels(torch, cr, lambda: cr.promote_batch(B), 5, flush, after=cr.free_batch)
    res["promote_batch"] = _kernel_line(rep, "bt_promote", 8 * 8192 * nk + B.array_pool_bytes + 9 * T + 8192 * T + 9 * T,
                                        t)
    for name, idx in (("multi_and_8_dense", list(range(8))), ("multi_and_4_dense_4_sparse", [0, 1, 2, 3, 8, 9, 10, 11])):
        r0 = cr.batch_multi_and(P, idx)
        n_common = r0.total_containers
        cr.free_batch(r0)
        t, rep = cold_time_and_kernels(torch, cr, lambda: cr.batch_multi_and(P, idx), 5, flush, after=cr.free_batch)
        nbytes = (len(idx) + 1) * 8192 * n_common + 9 * (len(idx) + 1) * n_common
        res[name] = dict(_kernel_line(rep, "bt_and", nbytes, t), n_common=n_common)
    words_each = Ub // 64
    d = torch.zeros(16 * words_each, dtype=torch.int64, device="cuda")
    cr.batch_decompress(B, d, words_each)  # first launch stays out of the timing
    torch.cuda.synchronize()
    t, rep = cold_time_and_kernels(torch, cr, lambda: cr.batch_decompress(B, d, words_each), 5, flush)
    res["decompress_batch"] = _kernel_line(rep, "bt_decompress", 8 * 8192 * nk + B.array_pool_bytes + 9 * T +
                                           16 * words_each * 8, t)
    del d
    nq = 100_000_000
    g = torch.Generator(device="cuda")
    g.manual_seed(71)
    q = torch.randint(0, Ub, (nq,), device="cuda", generator=g, dtype=torch.int64).to(torch.int32)
    qb = torch.randint(0, 16, (nq,), device="cuda", generator=g, dtype=torch.int64).to(torch.int32)
    out = torch.empty(nq, dtype=torch.uint8, device="cuda")
    cr.batch_contains(P, q, out, d_bitmap_idx=qb)
    torch.cuda.synchronize()
    t = cold_time(torch, lambda: cr.batch_contains(P, q, out, d_bitmap_idx=qb), 5, flush)
    res["contains_per_query_bitmap_promoted_Gqps"] = round(nq / t / 1e6, 2)
    t = cold_time(torch, lambda: cr.batch_contains(B, q, out, d_bitmap_idx=qb), 5, flush)
    res["contains_per_query_bitmap_mixed_Gqps"] = round(nq / t / 1e6, 2)
    v = cr.batch_make_view(P, 0)
    t = cold_time(torch, lambda: cr.batch_view_contains(v, q, out), 5, flush)
    res["view_contains_promoted_Gqps"] = round(nq / t / 1e6, 2)
    del q, qb, out
    cr.free_batch(P)
    cr.free_batch(B)
    log("batch api", {k: (v.get("frac_of_hbm_peak") if isinstance(v, dict) else v) for k, v in res.items()})
    return res


def sparse_arrays(cr, density, seed):
    """`density` of 2^30 as array containers through the packed upload
    (upload_from_ids builds all-bitmap above 1024 ids, whatever the threshold)."""
    import numpy as np
    ids = np.unique(np.random.default_rng(seed).integers(0, U, int(density * U), dtype=np.uint64))
    bounds = np.searchsorted(ids, np.arange((U >> 16) + 1, dtype=np.uint64) << np.uint64(16))
    conts = [(k, cr.TC_ARRAY, int(bounds[k + 1] - bounds[k]),
              (ids[bounds[k]:bounds[k + 1]] & np.uint64(0xFFFF)).astype(np.uint16))
             for k in range(U >> 16) if bounds[k + 1] > bounds[k]]
    return cr.upload_containers(conts, U, False, int(ids.size), cr.PROMOTE_KEEP_DEFAULT)


def conversions(torch, cr, flush, bitmaps):
    """decompress_to_bitset, enumerate_ids, promote_to_bitmap, the deep copy and
    cardinality on 2^30 bitmaps, cold.  Algorithmic bytes: the container payloads
    read (8192 B per bitmap, 2 B per array value), 9 B of metadata per container,
    plus what the call writes (4 B per bitset word, 8 B per id, 8192 B per promoted
    container, the copy; cardinality writes one count)."""
    res = {}
    for name, g in bitmaps.items():
        n = g.n_containers
        payload = 8192 * g.n_bitmap_containers + g.array_pool_bytes + g.run_pool_bytes + 9 * n
        kidx = 2 * (g.max_key + 1) if g.key_index else 0
        n_ids = g.total_cardinality
        words = torch.empty(U // 32, dtype=torch.int32, device="cuda")
        ids_out = torch.empty(n_ids, dtype=torch.int64, device="cuda")
        cases = {
            "decompress_to_bitset": (lambda: cr.decompress_to_bitset(g, words), payload + 4 * (U // 32),
                                     "cv_decompress", None),
            "enumerate_ids": (lambda: cr.enumerate_ids(g, ids_out), payload + 8 * n_ids, "cv_enum_write", None),
            "promote_to_bitmap": (lambda: cr.promote_to_bitmap(g),
                                  payload + 8192 * n + 9 * n + 2 * (g.max_key + 1), "cv_promote", True),
            "deep_copy": (lambda: cr.deep_copy(g), 2 * (payload + kidx), "cv_copy", True),
            "cardinality": (lambda: cr.cardinality(g), payload, "cv_card_sum", None),
        }
        r = {"n_containers": n, "n_bitmap": g.n_bitmap_containers, "n_array": g.n_array_containers, "ids": n_ids}
        for cname, (fn, nbytes, kname, frees) in cases.items():
            # a returned bitmap is freed outside the timed interval, so each call's
            # allocation comes from the library's cache, as in a steady state
            after = cr.free if frees else None
            x = fn()
            torch.cuda.synchronize()
            if frees:
                cr.free(x)
            t, rep = cold_time_and_kernels(torch, cr, fn, 5, flush, after=after)
            k_avg = rep.get(kname, (1, float("nan"), float("nan")))[2]
            r[cname] = {"algorithmic_bytes": nbytes, "api_ms": round(t, 4), "api_GBps": round(nbytes / t / 1e6, 1),
                        f"{kname}_ms": round(k_avg, 4), f"{kname}_GBps": round(nbytes / k_avg / 1e6, 1),
                        "frac_of_hbm_peak": round(nbytes / k_avg / 1e6 / HBM_PEAK_GBS, 4),
                        "kernels_ms": {k: round(v, 4) for k, v in kernel_medians(rep).items()},
                        "device_le_api": device_le_api(sum(kernel_medians(rep).values()), t)}
        # size-independent checks: enumerate gives ascending ids below U, and every
        # sampled id's bit is set in the bitset
        cr.enumerate_ids(g, ids_out)
        cr.decompress_to_bitset(g, words)
        torch.cuda.synchronize()
        assert bool((ids_out[1:] > ids_out[:-1]).all()) and int(ids_out[-1]) < U, "enumerate_ids not ascending"
        smp = ids_out[::997]
        bits = (words[smp >> 5].to(torch.int64) >> (smp & 31)) & 1
        assert bool((bits == 1).all()), "decompressed bitset misses an enumerated id"
        del words, ids_out, smp, bits
        torch.cuda.empty_cache()
        res[name] = r
        log("conversions", name, {k: v.get("frac_of_hbm_peak") for k, v in r.items() if isinstance(v, dict)})
    return res


TK_N, TK_Q, TK_DIM = 10_000_000, 1024, 128
FP32_MFMA_PEAK_TFLOPS = 157.3


def zipf_predicates(torch, targets, n_tags=10_000, per_vec=8, seed=52):
    """Per-vector tags ~ Zipf(1.1) over ranks 1..n_tags (8 per vector); for each
    target selectivity s, three predicates "has a tag in R_j" over disjoint random
    rank sets R_j, each sized so that P(pass) ~= s^(1/3).  Returns
    {s: (masks [3 x N bool], achieved selectivity of the AND)}."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    ranks = torch.arange(1, n_tags + 1, device="cuda", dtype=torch.float64)
    w = ranks.pow(-1.1)
    w /= w.sum()
    cdf = torch.cumsum(w, 0)
    u = torch.rand((TK_N, per_vec), device="cuda", generator=g, dtype=torch.float64)
    tags = torch.searchsorted(cdf, u).clamp_(max=n_tags - 1)  # 0-based rank
    del u
    out = {}
    for s in targets:
        perm = torch.randperm(n_tags, device="cuda", generator=g)
        p1 = s ** (1.0 / 3.0)
        w_star = 1.0 - (1.0 - p1) ** (1.0 / per_vec)  # tag mass a rank set needs
        masks, start = [], 0
        for _ in range(3):
            cum = torch.cumsum(w[perm[start:]], 0)
            take = int(torch.searchsorted(cum, torch.tensor([w_star], device="cuda", dtype=torch.float64)).item()) + 1
            sel = torch.zeros(n_tags, dtype=torch.bool, device="cuda")
            sel[perm[start:start + take]] = True
            start += take
            masks.append(sel[tags].any(dim=1))
        both = masks[0] & masks[1] & masks[2]
        out[s] = (masks, float(both.float().mean().item()))
    del tags
    return out


def topk_secondary(torch, cr, no_cpu):
    """Fused filtered brute-force top-k (config 5): 10M x 128 fp32 base ~ N(0,1),
    1024 queries, squared L2, k in {10, 100}, filter = multi_and of three Zipf-tag
    predicates at selectivities 0.1/1/10/50%, plus the unfiltered control."""
    g = torch.Generator(device="cuda")
    g.manual_seed(50)
    base = torch.randn((TK_N, TK_DIM), device="cuda", dtype=torch.float32, generator=g)
    g.manual_seed(51)
    queries = torch.randn((TK_Q, TK_DIM), device="cuda", dtype=torch.float32, generator=g)
    preds = zipf_predicates(torch, (0.001, 0.01, 0.1, 0.5))
    out = {"base": f"{TK_N} x {TK_DIM} fp32 N(0,1)", "queries": TK_Q}
    runs = [("unfiltered", None, 1.0)]
    for s, (masks, achieved) in preds.items():
        gs = [cr.upload_from_device_ids(torch.nonzero(m).flatten().to(torch.int32), TK_N) for m in masks]
        f = cr.multi_and(gs)
        for x in gs:
            cr.free(x)
        runs.append((f"sel_{s:g}", f, achieved))
    del preds
    for k in (10, 100):
        dist = torch.empty((TK_Q, k), device="cuda", dtype=torch.float32)
        ids = torch.empty((TK_Q, k), device="cuda", dtype=torch.int64)
        for name, f, sel in runs:
            cr.topk_filtered(base, queries, k, f, dist, ids)
            torch.cuda.synchronize()
            cr.timing_enable(True)
            ts = []
            for _ in range(3):
                t0 = time.perf_counter()
                cr.topk_filtered(base, queries, k, f, dist, ids)
                torch.cuda.synchronize()
                ts.append((time.perf_counter() - t0) * 1e3)
            rep = cr.timing_report()
            cr.timing_enable(False)
            t = median(ts)
            n_pass = TK_N if f is None else int(round(sel * TK_N))
            flops = 2.0 * TK_DIM * n_pass * TK_Q
            # the MFMA kernels: tk_dist (list path) and tk_pairs (small sets' estimates, larger sets' seed rows)
            kms = sum(v[2] for kk, v in rep.items() if kk in ("tk_dist", "tk_pairs"))
            ok = bool((ids[:, 0] >= 0).all().item()) and bool((dist[:, 1:] >= dist[:, :-1]).all().item())
            out[f"k{k}_{name}"] = {
                "selectivity": round(sel, 6), "ms": round(t, 3), "qps": round(TK_Q / (t / 1e3), 1),
                "mfma_kernels_ms": round(kms, 3),
                "mfma_tflops": round(flops / (kms / 1e3) / 1e12, 2),
                "mfma_frac_fp32_peak": round(flops / (kms / 1e3) / 1e12 / FP32_MFMA_PEAK_TFLOPS, 4),
                "kernels_ms": {kk: round(v, 4) for kk, v in kernel_medians(rep).items()}, "sane": ok,
                "device_le_api": device_le_api(sum(kernel_medians(rep).values()), t),
            }
            log(f"topk k={k} {name}", out[f"k{k}_{name}"]["ms"], "ms", out[f"k{k}_{name}"]["mfma_frac_fp32_peak"])
    for _, f, _ in runs:
        if f is not None:
            cr.free(f)
    if not no_cpu:
        # Bounded CPU samples of the same workload (unfiltered): the blocked fp32
        # brute-force scan (orc_cpu_topk_fp32) over all 10M base vectors for 64
        # queries at every host thread, and over 1M base vectors for 16 queries at
        # one thread (QPS scaled to the 10M base).
        import orc
        nt = cpu_threads()
        hb = base.cpu().numpy()
        hq = queries[:64].cpu().numpy()
        cpu = {"kind": "port", "cores": nt, "cpu": cpu_info()}
        import numpy as np
        agree = True
        for k in (10, 100):
            tn, d_, i_ = orc.cpu_topk_fp32(hb, hq, k, None, nt)
            t1, _, _ = orc.cpu_topk_fp32(hb[:1_000_000], hq[:16], k, None, 1)
            cpu[f"k{k}_qps_{nt}t"] = round(hq.shape[0] / tn, 2)
            cpu[f"k{k}_qps_1t"] = round(16 / (t1 * TK_N / 1_000_000), 3)
            # the GPU's answer for the same 64 queries equals the CPU scan's
            gd = torch.empty((64, k), device="cuda", dtype=torch.float32)
            gi = torch.empty((64, k), device="cuda", dtype=torch.int64)
            cr.topk_filtered(base, queries[:64], k, None, gd, gi)
            torch.cuda.synchronize()
            agree &= bool(np.allclose(gd.cpu().numpy(), d_, rtol=1e-4, atol=0))
            agree &= all(set(a) == set(b) for a, b in zip(gi.cpu().numpy().tolist(), i_.tolist()))
        cpu["gpu_answers_equal_cpu_scan"] = agree
        cpu["sample"] = (f"orc_cpu_topk_fp32 (blocked fp32 scan, direct squared L2, AVX2) unfiltered: 10M x 128 "
                         f"base x 64 queries at {nt} threads; 1M x 128 x 16 queries at 1 thread, scaled to 10M")
        out["cpu_baseline"] = cpu
        del hb
    del base, queries
    torch.cuda.empty_cache()
    return out


def cpu_baseline(ids_host):
    """The CPU upload of the headline ids: a threaded bucket build
    (orc_cpu_upload_ids) on all 100M ids at every host thread (`value`, median
    of 3), and on the first 10M at one thread; the reference's own CPU
    algorithm (sort + unique + bitmap build, one thread: orc_upload_from_ids)
    on the first 10M.  The 10M samples are scaled x10 to the 100M workload."""
    import ctypes as C

    import numpy as np
    import orc
    lib = orc.cpu_lib()
    full = np.ascontiguousarray(ids_host, dtype=np.uint32)
    s = full[:10_000_000]
    scale = N_IDS / s.size

    def sort_based():
        c = orc._OrcRoaring()
        t0 = time.perf_counter()
        rc = lib.orc_upload_from_ids(s.ctypes.data, s.size, U, orc.PROMOTE_AUTO, orc.DEFAULT_L2, C.byref(c))
        dt = time.perf_counter() - t0
        assert rc == 0
        n_c = c.n_containers
        lib.orc_free(C.byref(c))
        return dt, n_c
    t_sort, n_c = sorted(sort_based() for _ in range(3))[1]
    nt = cpu_threads()
    runs = []
    for _ in range(3):
        t, r = orc.cpu_upload_ids(s, U, 1)
        assert r.n_containers == n_c
        runs.append(t)
    t1 = sorted(runs)[1]
    runs = []
    for _ in range(3):
        t, r = orc.cpu_upload_ids(full, U, nt)
        assert r.n_containers == 16384
        runs.append(t)
    tn = sorted(runs)[1]
    return {"value": round(tn * 1e3, 1), "unit": "ms", "cores": nt, "kind": "port",
            "sample": f"all {full.size // 1_000_000}M headline ids: orc_cpu_upload_ids (bucket partition by key "
                      f"range + bit set + popcount, the same all-bitmap layout) at {nt} threads, median of 3",
            "one_thread_ms": round(t1 * 1e3 * scale, 1),
            "one_thread_sample": f"the first {s.size // 1_000_000}M ids, scaled x{scale:g}",
            "reference_algorithm_one_thread_ms": round(t_sort * 1e3 * scale, 1),
            "reference_algorithm": "orc_upload_from_ids: qsort + unique + bitmap build, the reference's CPU "
                                   "pipeline (std::sort + unique + upload, bench/bench_upload_scale.cu:102-125)",
            "isa": orc.cpu_isa(), "cpu": cpu_info()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-topk", action="store_true")
    ap.add_argument("--secondary-out", default=None,
                    help="where the secondary sections' JSON goes (default gpurun_out/bench_secondary.json)")
    ap.add_argument("--sections", default=",".join(SECTIONS),
                    help="comma-separated secondary sections to run (default: all of " + ",".join(SECTIONS) + ")")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the sharded design is "
              f"described, not run, in this build.", file=sys.stderr)
        sys.exit(2)
    rank = int(os.environ.get("RANK", "0"))

    import torch

    import curoaring as cr
    cr.load()
    torch.cuda.set_device(0)
    log("generating ids")
    d_ids = make_ids(torch)
    torch.cuda.synchronize()
    flush = torch.zeros(512 << 20, dtype=torch.uint8, device="cuda")

    for _ in range(args.warmup):
        g = cr.upload_from_device_ids(d_ids, U)
        cr.free_async(g)
    torch.cuda.synchronize()
    log("warmup done")

    # Timed steps, cold: before each step a 512 MiB read evicts the 256 MB
    # Infinity Cache (outside the step's interval); each step is bracketed by a
    # device synchronisation on both sides.  HIP events around every
    # EVENT_EVERY-th launch of each kernel give the device time of the path
    # (the markers cost queue time, so sampling keeps the steps close to
    # untimed ones).
    cr.timing_enable(True, every=EVENT_EVERY)
    step_ms = []
    last = None
    for k in range(args.steps):
        evict(flush)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        g = cr.upload_from_device_ids(d_ids, U)
        if k == args.steps - 1:
            last = g
        else:
            cr.free_async(g)
        torch.cuda.synchronize()
        step_ms.append((time.perf_counter() - t0) * 1e3)
    rep = cr.timing_report()
    cr.timing_enable(False)
    ms_per_step = sum(step_ms) / len(step_ms)
    n_c = last.n_containers
    total = last.total_cardinality
    ok = (n_c == 16384 and total == N_DISTINCT and not last.negated and last.max_key == 16383)
    cr.free(last)
    if not ok:
        log("PROPERTY CHECK FAILED", n_c, total)
        sys.exit(1)
    log("timed steps done (cold)", round(ms_per_step, 4), "ms/step")

    # The same steps back to back with no eviction (warm), reported beside.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        g = cr.upload_from_device_ids(d_ids, U)
        cr.free_async(g)
    torch.cuda.synchronize()
    warm_ms = (time.perf_counter() - t0) * 1e3 / args.steps

    per_kernel = {k: v[1] / v[0] for k, v in rep.items() if not k.startswith("host:")}
    per_kernel_median = kernel_medians(rep)
    host_ms = {k[5:]: round(v[1] / args.steps, 4) for k, v in rep.items() if k.startswith("host:")}
    path = [k for k in UPLOAD_PATH if k in per_kernel]
    dev_ms = sum(per_kernel[k] for k in path)  # each kernel launches once per step
    dom = max(path, key=lambda k: per_kernel[k])
    path_bytes = 4 * N_IDS + 8192 * n_c + 9 * n_c + 2 * (16383 + 1)
    achieved = path_bytes / dev_ms / 1e6
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic_upload_ids.json")
    if os.path.exists(tpath):
        try:
            tj = json.load(open(tpath))
            traffic = sum(int(tj[k]) for k in path)
        except Exception:
            traffic = None
    kernels = {}
    for k in path:
        kb = upload_kernel_bytes(k, N_IDS, n_c, 16383)
        kernels[k] = {"mean_ms": round(per_kernel[k], 5), "median_ms": round(per_kernel_median[k], 5),
                      "launches": rep[k][0]}
        if kb:
            kernels[k].update({"bytes": kb, "frac": round(kb / per_kernel[k] / 1e6 / HBM_PEAK_GBS, 4)})

    # BASELINE configs[1] names the three threshold variants: above 1024 ids the
    # reference builds all-bitmap whatever the threshold (src/upload_ids.cu:573-587),
    # so each must give the AUTO result; each is timed cold like the headline.
    variants = {}
    for tname, thr in (("AUTO", cr.PROMOTE_AUTO), ("KEEP_DEFAULT", cr.PROMOTE_KEEP_DEFAULT),
                       ("ALL", cr.PROMOTE_ALL)):
        t = cold_time(torch, lambda: cr.upload_from_device_ids(d_ids, U, thr), 7, flush, after=cr.free_async)
        g = cr.upload_from_device_ids(d_ids, U, thr)
        same = (g.n_containers, g.total_cardinality, g.n_bitmap_containers, g.max_key) == (n_c, total, n_c, 16383)
        cr.free(g)
        variants[tname] = {"ms": round(t, 4), "same_result": same}
        if not same:
            log("THRESHOLD VARIANT DIFFERS", tname)
            sys.exit(1)

    result = {
        "metric": "upload ms @100M IDs",
        "value": round(ms_per_step, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32",
        "data": "synthetic: 90M distinct pseudo-random ids (bijective 30-bit hash) + 10M duplicates, shuffled, "
                "device-resident",
        "config": {"workload": "upload_from_ids, 100M unsorted u32 ids (~10% duplicates), universe 2^30, "
                               "PROMOTE_AUTO (BASELINE configs[1], uniform variant)",
                   "universe": U, "n_ids": N_IDS, "distinct": N_DISTINCT, "parallelism": "single GPU"},
        "timing": "cold: a 512 MiB read evicts the Infinity Cache before each step, outside its interval; "
                  "value = mean of the steps, each bracketed by device synchronisation",
        "warm_ms_per_step": round(warm_ms, 4),
        "ids_per_s": round(N_IDS / (ms_per_step / 1e3), 1),
        "roofline": {"bound": "hbm", "kernel": "upload_from_ids path (" + " + ".join(path) + ")",
                     "dominant_kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "algorithmic_bytes_per_launch": path_bytes,
                     "algorithmic_bytes_formula": "4 N + 8192 n_c + 9 n_c + 2 (max_key + 1)",
                     "mean_launch_ms": round(dev_ms, 5), "events_every": EVENT_EVERY,
                     "end_to_end_frac": round(path_bytes / ms_per_step / 1e6 / HBM_PEAK_GBS, 4)},
        "kernels": kernels,
        "host_ms_per_step": host_ms,
        "threshold_variants_ms": variants,
    }
    # Achievable-bandwidth reference: a plain 1 GiB device copy (also the known-size
    # kernel that calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE).
    src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    copy_ms = e0.elapsed_time(e1) / 5
    result["copy_1GiB"] = {"ms": round(copy_ms, 4), "GBps_read_plus_write": round(2 * (1 << 30) / copy_ms / 1e6, 1)}
    del src, dst
    # PCIe-inclusive rate: the reference's entry point takes pageable host ids and
    # copies them to the device first.  Reported beside the headline, never as it.
    h_ids = d_ids.cpu().numpy().view("uint32")
    g = cr.upload_from_ids(h_ids, U)
    cr.free(g)
    host_ms = []
    for _ in range(3):
        t0 = time.perf_counter()
        g = cr.upload_from_ids(h_ids, U)
        host_ms.append((time.perf_counter() - t0) * 1e3)
        cr.free(g)
    result["upload_from_host_ids"] = {"ms": round(median(host_ms), 3),
                                      "note": "cr_upload_from_ids on 100M pageable host ids, H2D included"}
    del h_ids
    result["device"] = {"l2_bytes": cr.device_l2_bytes(), "auto_threshold_2^30": cr.resolve_auto_threshold(U)}
    log("host-ids upload", result["upload_from_host_ids"], result["device"])
    if rank == 0 and not args.no_cpu:
        log("cpu baseline (all 100M ids at every thread; 10M-id samples at one thread)")
        sample = d_ids.cpu().numpy().view("uint32")
        result["cpu_baseline"] = cpu_baseline(sample)
        log("cpu baseline", result["cpu_baseline"])
    sec = None
    if not args.no_secondary:
        del d_ids
        torch.cuda.empty_cache()
        sections = set(args.sections.split(","))
        sec = secondary(torch, cr, flush, args.no_cpu, sections)
        if not args.no_topk and "topk" in sections:
            del flush
            torch.cuda.empty_cache()
            sec["topk_10M_x128_q1024"] = topk_secondary(torch, cr, args.no_cpu)
        sec["device_gt_api"] = DEVICE_GT_API
        # The full secondary tree (tens of KB) goes to its own file; the stdout
        # line carries the headline and a few figures from it.
        out_path = args.secondary_out or os.path.join(ROOT, "gpurun_out", "bench_secondary.json")
        try:
            os.makedirs(os.path.dirname(out_path), exist_ok=True)
            with open(out_path, "w") as f:
                json.dump(sec, f, indent=1)
            result["secondary_file"] = os.path.relpath(out_path, ROOT)
        except OSError as e:
            log("could not write the secondary sections:", e)
        result["secondary_highlights"] = highlights(sec)
        result["device_time_exceeds_api_lines"] = len(DEVICE_GT_API)
    line = json.dumps(result, separators=(",", ":"))
    if len(line) > 6000:  # keep the driver-parsed line small
        result.pop("secondary_highlights", None)
        line = json.dumps(result, separators=(",", ":"))
    print(line, flush=True)


def highlights(sec):
    """A few figures of the secondary sections, for the headline line (each is
    taken only if its section ran)."""
    h = {}

    def take(name, fn):
        try:
            h[name] = fn()
        except (KeyError, TypeError, ValueError, ZeroDivisionError):
            pass
    c3 = sec.get("config3_point_queries_2^30", {})
    take("queries_10pct_uniform_partitioned_Gqps", lambda: c3["density_10pct"]["compressed_uniform_partitioned_Gqps"])
    take("queries_10pct_uniform_partitioned_frac_18B",
         lambda: c3["density_10pct"]["compressed_uniform_partitioned_frac_hbm_18B"])
    take("queries_10pct_uniform_contains_Gqps", lambda: c3["density_10pct"]["compressed_uniform_contains_Gqps"])
    take("queries_1pct_uniform_partitioned_Gqps", lambda: c3["density_1pct"]["compressed_uniform_partitioned_Gqps"])
    c2 = sec.get("config2_set_ops_2^30", {})
    for pair in ("BB'_AND", "AB_OR", "AB_AND", "BC_OR", "AC_OR", "CC'_AND", "AA'_AND"):
        take(f"setop_{pair}_exec_frac", lambda p=pair: c2[p]["exec_frac_of_hbm_peak"])
        take(f"setop_{pair}_api_ms", lambda p=pair: c2[p]["api_ms"])
    take("multi_and_k8_fused_frac", lambda: c2["multi_and_k8_fused_all_bitmap"]["mand_and_frac_of_hbm_peak"])
    take("multi_and_k8_fused_api_ms", lambda: c2["multi_and_k8_fused_all_bitmap"]["api_ms"])
    uv = sec.get("upload_variants_2^30", {})
    take("upload_clustered_100M_ms", lambda: uv["ids_clustered_100M"]["ms"])
    take("upload_bitset_0.1pct_ms", lambda: uv["bitset_0.1pct"]["ms"])
    take("upload_bitset_0.1pct_frac", lambda: uv["bitset_0.1pct"]["frac_of_hbm_peak"])
    tk = sec.get("topk_10M_x128_q1024", {})
    for case in ("k10_unfiltered", "k10_sel_0.1", "k10_sel_0.01", "k10_sel_0.001", "k100_sel_0.1"):
        take(f"topk_{case}_ms", lambda c=case: tk[c]["ms"])
        take(f"topk_{case}_mfma_frac", lambda c=case: tk[c]["mfma_frac_fp32_peak"])
    cv = sec.get("conversions_2^30", {})
    take("decompress_10pct_frac", lambda: cv["dense_10pct_bitmap"]["decompress_to_bitset"]["frac_of_hbm_peak"])
    return h


if __name__ == "__main__":
    main()

"""Benchmark of the search hot path on one MI355X.

The default run measures all five BASELINE configs, one after the other, and
prints ONE JSON line: the headline at the top level and
configs 1, 3, 4 and 5 under "configs", each with its own value, roofline,
host-buffer rate, CPU baseline and exact-oracle check.

Headline workload: flat cosine search, 1,000,000 x 768
fp32 rows (i.i.d. N(0,1), each L2-normalised), 10,000 queries drawn the same
way, k = 100, distance 1 - q.x.  One step = one vsk_search_flat call over all
10,000 queries with the database and the queries already in HBM.

The configs (also runnable alone with ``--config``):

* ``c1`` flat L2^2, 10,000 x 128, 100 queries, k = 10 (latency-bound);
* ``c3`` IVF-Flat L2, 1M x 128 from a 4,096-Gaussian mixture, nlist 4096,
  nprobe 32, 10,000 queries, k = 10 (one step = one vsk_ivf_search);
* ``c4`` int8 SQ scan, 10M x 128 codes, 1,000 queries, k = 100;
* ``c5`` PQ M=16 x 256 ADC over 10M codes, top-1000, exact L1 re-rank to
  k = 100 (one step = one vsk_pq_search);
* ``c3train`` IVF coarse training on config 3's data: k-means of 1M x 128
  rows into 4,096 clusters, 10 Lloyd iterations per step (vsk_kmeans),
  reported as row-iterations/s;
* ``c4bin`` binary quantization of config 4's data (10M x 128 -> 16-byte
  codes), 1,000 queries, Hamming top-100 (vsk_bin_search).

Per config: QPS (value, inputs and outputs resident in HBM), the roofline of
the dominant kernel (algorithmic FLOP/OP or bytes per (query, row) pair the
library counted for that kernel's launches, over its HIP-event time on the
library's stream), the same call on host buffers (``host_io_inclusive``, the
PCIe-inclusive rate, never the value), and a CPU baseline: the oracle on this
host's cores over the first queries of the same workload, its CPU model,
and the GPU's results on those queries checked against it bit for bit
(``exact_oracle_check``).  ``traffic`` is the kernel's HBM bytes per launch
looked up in profiles/hbm_traffic.json (rocprofv3 FETCH_SIZE/WRITE_SIZE
passes, scaled by a plain-copy calibration; ``traffic_source`` names the
commit) when that file holds an entry for this kernel and workload, else null.

    python bench.py [--config all|c1..c5|...] [--steps K] [--warmup W] [--gpus 1]
                    [--no-cpu] [--no-host-io]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32_MFMA_TFLOPS = 157.3  # MI355X dense fp32 matrix, datasheet
PEAK_FP32_VALU_TFLOPS = 157.3   # fp32 vector, packed FMA
PEAK_FP32_VALU_ISSUE_TOPS = 39.3  # 256 CU x 4 SIMD x 16 lanes x 2.4 GHz, one op per lane-cycle
PEAK_BF16_MFMA_TFLOPS = 2500.0  # MI355X dense bf16 matrix, datasheet
PEAK_INT8_MFMA_TOPS = 5000.0  # MI355X dense int8 matrix, datasheet
PEAK_HBM_GBPS = 8000.0  # MI355X HBM3E, datasheet
PEAK_LDS_LOOKUPS = 256 * 64 * 2.4e9  # 4-byte LDS reads/s, 64 banks x 256 CUs
# the same ceilings re-measured on the device at start (vsk_measure_peaks):
# each roofline also reports its fraction of these
MEASURED_PEAKS = {}

DEFAULT_STEPS = {"c1": (200, 20), "c2": (5, 1), "c3": (5, 1), "c4": (5, 1), "c5": (5, 1),
                 "c5lut": (3, 1),
                 "c3train": (2, 1), "c4bin": (5, 1), "c3sq8": (5, 1), "c3pq": (5, 1),
                 "all": (20, 5)}
# the BASELINE configs the default run measures; the first is the headline
BASELINE_CONFIGS = ("c2", "c1", "c3", "c4", "c5")
# measured after them in the default run: config 5 through the LUT scan over
# the codes alone (no decoded plane), beside the screened line
EXTRA_CONFIGS = ("c5lut",)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--config", default="all", choices=sorted(DEFAULT_STEPS),
                   help="all (default): the five BASELINE configs, config 2 as the "
                        "headline and the others under 'configs'")
    p.add_argument("--steps", type=int, default=None)
    p.add_argument("--warmup", type=int, default=None)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-host-io", action="store_true",
                   help="skip the host-buffer (PCIe-inclusive) timing")
    p.add_argument("--cpu-seconds", type=float, default=None,
                   help="target length of each CPU baseline sample (default 15 s, 10 s "
                        "per config for --config all)")
    p.add_argument("--kmeans-init", default="random", choices=["random", "kmeans++"],
                   help="c3train: the seeding (random rows or k-means++ on the device)")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="only run a plain device copy of MIB MiB 3 times (the "
                        "reference kernel for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    a = p.parse_args()
    s, w = DEFAULT_STEPS[a.config]
    a.steps = s if a.steps is None else a.steps
    a.warmup = w if a.warmup is None else a.warmup
    if a.cpu_seconds is None:
        a.cpu_seconds = 10.0 if a.config == "all" else 15.0
    return a


def cpu_model():
    """The host CPU as /proc/cpuinfo names it (vendor, family, model)."""
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if ":" in line:
                    k, v = (t.strip() for t in line.split(":", 1))
                    info.setdefault(k, v)
                if not line.strip() and info:
                    break
    except OSError:
        return "unknown"
    return (f"{info.get('model name', 'unknown')} ({info.get('vendor_id', '?')}, family "
            f"{info.get('cpu family', '?')}, model {info.get('model', '?')})")


def progress(msg):
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def copy_calibration(mib):
    """A plain copy kernel of known size: reads and writes mib MiB."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.ones(n, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_mib": mib, "bytes_read": n * 4, "bytes_written": n * 4}))


def host_threads():
    return len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()


def cpu_sample(run, nq_total, target_s, threads):
    """Times ``run(m)`` (the oracle over the first m queries, all threads):
    a warm-up and a probe round of ``threads`` queries, then samples sized
    from the last measured rate until one lasts at least half of target_s
    (the whole set repeated when it is quicker).  A probe underestimates the
    rate of a large sample (the flat oracle keeps one thread per 4-query
    group busy), hence the re-sizing.  Returns (queries/s, m, repeats,
    seconds, result of the last call)."""
    m0 = min(nq_total, threads)
    run(m0)
    t0 = time.perf_counter()
    res = run(m0)
    el = time.perf_counter() - t0
    m, reps = m0, 1
    for _ in range(4):
        if el >= 0.5 * target_s:
            break
        per_q = max(el, 1e-4) / (m * reps)
        want = max(1, int(target_s / per_q))
        nm = min(nq_total, want)
        nreps = max(1, want // nq_total) if nm == nq_total else 1
        if (nm, nreps) == (m, reps):
            break
        m, reps = nm, nreps
        t0 = time.perf_counter()
        for _ in range(reps):
            res = run(m)
        el = time.perf_counter() - t0
    return m * reps / el, m, reps, el, res


def id_agreement(gi, oi):
    """Fraction of the CPU's top-k ids that the GPU also returned."""
    hits = sum(len(set(a) & set(b)) for a, b in zip(gi.tolist(), oi.tolist()))
    return hits / max(1, oi.size)


# ---------------------------------------------------------------- workloads

def gen_flat(n, d, nq, normalise, dev):
    import torch

    g = torch.Generator(device=dev)
    g.manual_seed(1)
    x = torch.randn(n, d, generator=g, device=dev)
    g.manual_seed(2)
    q = torch.randn(nq, d, generator=g, device=dev)
    if normalise:
        x /= x.norm(dim=1, keepdim=True)
        q /= q.norm(dim=1, keepdim=True)
    return x, q


def gen_mixture(n, d, ncent, nq, dev, jitter=True):
    """centres ~ N(0, 4 I) (seed 3), centre index uniform (seed 5), points =
    centre + 0.5 N(0, I) (rows seed 1, queries seed 2), centroids = centres +
    0.1 N(0, I) (seed 4)."""
    import torch

    g = torch.Generator(device=dev)
    g.manual_seed(3)
    cent = 2.0 * torch.randn(ncent, d, generator=g, device=dev)
    g.manual_seed(5)
    a = torch.randint(0, ncent, (n,), generator=g, device=dev)
    qa = torch.randint(0, ncent, (nq,), generator=g, device=dev)
    g.manual_seed(1)
    x = cent[a] + 0.5 * torch.randn(n, d, generator=g, device=dev)
    del a
    g.manual_seed(2)
    q = cent[qa] + 0.5 * torch.randn(nq, d, generator=g, device=dev)
    c = None
    if jitter:
        g.manual_seed(4)
        c = cent + 0.1 * torch.randn(ncent, d, generator=g, device=dev)
    return x, q, c


def exact_check(gd, gi, od, oi, m):
    """The GPU's first m results against the oracle's, bit for bit."""
    import numpy as np

    gd, gi = np.asarray(gd)[:m], np.asarray(gi)[:m]
    same_d = gd.view(np.uint32) == np.asarray(od).view(np.uint32) if gd.dtype == np.float32 \
        else gd == np.asarray(od)
    return {"queries": int(m), "ids_equal": bool((gi == np.asarray(oi)).all()),
            "distances_bitwise_equal": bool(same_d.all())}


def probed_pairs(idx, q, nprobe):
    """(query, row) pairs an IVF search scores: the sizes of each query's
    probed lists, summed over the queries."""
    sizes = idx.list_sizes()
    probes = idx.probe(q, nprobe)
    probes = probes.cpu().numpy() if hasattr(probes, "cpu") else np.asarray(probes)
    return int(sizes[probes[probes >= 0]].sum())


def setup(c, a, ctx, dev):
    """Builds the resident index for config c; returns (spec, step, cpu_leg,
    host_step): cpu_leg(target_s) gives (baseline dict, agreement), and
    host_step (or None) runs the same call on host buffers (queries read
    from and results written to host memory, the PCIe-inclusive case)."""
    import numpy as np
    import torch

    from vectorstorekit_amd import _lib as L
    from vectorstorekit_amd import (IVFConfiguration, IVFIndex, ProductQuantizer,
                                    ScalarQuantizer, SQ8Database, VectorDatabase)

    lib = ctx.lib
    if c in ("c1", "c2"):
        n, d, nq, k = (10_000, 128, 100, 10) if c == "c1" else (1_000_000, 768, 10_000, 100)
        metric = L.METRIC_L2SQ if c == "c1" else L.METRIC_COSINE_NORMALIZED
        x, q = gen_flat(n, d, nq, c == "c2", dev)
        db = VectorDatabase(ctx, x)
        dist = torch.empty(nq, k, device=dev)
        ids = torch.empty(nq, k, dtype=torch.int64, device=dev)

        def step():
            ctx.check(lib.vsk_search_flat(ctx.handle, db.handle, q.data_ptr(), nq, k, metric,
                                          dist.data_ptr(), ids.data_ptr()))

        qhost = q.cpu().numpy()
        hd, hi = np.empty((nq, k), np.float32), np.empty((nq, k), np.int64)

        def host_step():
            ctx.check(lib.vsk_search_flat(ctx.handle, db.handle, qhost.ctypes.data, nq, k,
                                          metric, hd.ctypes.data, hi.ctypes.data))

        def cpu_leg(target_s):
            from oracle import oracle as O
            qh = qhost
            th = host_threads()
            # the exact restatement (dimension-order sums, rows side by side
            # in SIMD lanes) over its resident database: the timed port is
            # also the parity check
            cdb = O.FlatDB(x.cpu().numpy(), threads=th)
            qps, m, reps, el, (od, oi) = cpu_sample(
                lambda m: cdb.search(qh[:m], k, metric, threads=th), nq, target_s, th)
            del cdb
            gd, gi = dist.cpu().numpy(), ids.cpu().numpy()
            return ({"value": qps, "unit": "queries/s", "cores": th, "kind": "port",
                     "cpu": cpu_model(),
                     "sample": f"first {m} of {nq} queries against all {n} rows, "
                               f"{reps} pass(es) ({el:.1f} s), exact dimension-order sums",
                     "exact_oracle_check": exact_check(gd, gi, od, oi, m)},
                    id_agreement(gi[:m], oi))

        spec = {
            "metric": ("QPS @k=100, 1M x 768 fp32 flat cosine" if c == "c2"
                       else "QPS @k=10, 10k x 128 fp32 flat L2^2"),
            "workload": (f"flat-cosine-1Mx768-q10000-k100 (BASELINE config 2)" if c == "c2"
                         else "flat-l2sq-10000x128-q100-k10 (BASELINE config 1)"),
            "config": {"n": n, "d": d, "nq": nq, "k": k,
                       "metric": "1 - q.x" if c == "c2" else "sum (q-x)^2"},
            "data": ("synthetic: N(0,1) rows and queries (torch Philox seeds 1, 2)"
                     + (", L2-normalised" if c == "c2" else "")),
            "dtype": "f32", "nq": nq, "n": n, "d": d,
            "kernels": [("flat_screen_filter", "k_flat_screen<FILTER>", "mfma_bf16"),
                        ("flat_screen_dense", "k_flat_screen<DENSE>", "mfma_bf16"),
                        # small problems: the exact sequential scan alone
                        ("flat_valu_dense", "k_flat_valu<DENSE> (exact, dimension order)",
                         "valu_l2" if c == "c1" else "valu_dot"),
                        ("flat_bf16x3_filter", "k_flat_bf16x3<FILTER>", "mfma"),
                        ("flat_bf16x3_dense", "k_flat_bf16x3<DENSE>", "mfma"),
                        ("flat_mfma_filter", "k_flat_mfma<FILTER>", "mfma32"),
                        ("flat_mfma_dense", "k_flat_mfma<DENSE>", "mfma32")],
            "keep": (db, x, q, dist, ids),
        }
        return spec, step, cpu_leg, host_step

    if c == "c3train":
        # IVF coarse training at config 3's scale: one step = one vsk_kmeans
        # call, 10 Lloyd iterations (tolerance 0 never stops early) from 4,096
        # seeded random rows
        from vectorstorekit_amd.clustering import (INIT_PLUSPLUS, INIT_RANDOM,
                                                   vsk_kmeans_result)
        n, d, ncent, iters = 1_000_000, 128, 4096, 10
        init = INIT_PLUSPLUS if a.kmeans_init == "kmeans++" else INIT_RANDOM
        x, _, _ = gen_mixture(n, d, ncent, 1, dev, jitter=False)
        cent = torch.empty(ncent, d, device=dev)
        assign = torch.empty(n, dtype=torch.int32, device=dev)
        res = vsk_kmeans_result()
        import ctypes

        def step():
            ctx.check(lib.vsk_kmeans(ctx.handle, x.data_ptr(), n, d, ncent, None, init,
                                     None, ctypes.c_uint64(7), iters, 0.0, cent.data_ptr(),
                                     assign.data_ptr(), ctypes.byref(res)))

        def cpu_leg(target_s):
            from oracle import oracle as O
            th = host_threads()
            xh = x.cpu().numpy()
            # the oracle's Lloyd loop on a row sample: 2 iterations from the
            # GPU's final centroids (an assignment of m x 4096 pairs and the
            # update, per iteration)
            ch = cent.cpu().numpy()
            m = 4096
            t0 = time.perf_counter()
            O.kmeans_cluster(xh[:m], ncent, init_method="custom", init=ch, max_iter=1, tol=0.0,
                             threads=th)
            per = time.perf_counter() - t0
            m = int(min(n, max(4096, m * target_s / 2 / max(per, 1e-3))))
            t0 = time.perf_counter()
            O.kmeans_cluster(xh[:m], ncent, init_method="custom", init=ch, max_iter=2, tol=0.0,
                             threads=th)
            el = time.perf_counter() - t0
            return ({"value": m * 2 / el, "unit": "row-iterations/s", "cores": th,
                     "kind": "port", "cpu": cpu_model(),
                     "sample": f"first {m} of {n} rows, 2 Lloyd iterations against "
                               f"{ncent} centroids ({el:.1f} s)"}, 1.0)

        spec = {
            "metric": "k-means row-iterations/s, 1M x 128, k = 4096 (IVF training at "
                      "config 3's scale)",
            "workload": "kmeans-1Mx128-k4096-iter10 (IVF coarse training, BASELINE config 3 data)",
            "config": {"n": n, "d": d, "k": ncent, "iterations": iters,
                       "init": f"{a.kmeans_init} (seed 7)"},
            "data": "synthetic: 4,096-Gaussian mixture, centres 2 N(0,I) (seed 3), points "
                    "centre + 0.5 N(0,I) (seeds 5, 1)",
            "dtype": "f32", "nq": n, "n": ncent, "d": d,
            "units_per_step": n * iters, "unit": "row-iterations/s",
            "kernels": [("kmeans_plusplus", "k-means++ seeding (k_kpp_update / blocksum / "
                         "pick per centroid)", "kpp"),
                        ("flat_valu_argmin", "k_flat_valu<ARGMIN> (exact sqrt-L2, dimension "
                         "order)", "valu_l2"),
                        ("flat_screen_top2", "k_flat_screen<TOP2> (bf16 screen, smallest two per "
                         "row)", "mfma_bf16")],
            "keep": (x, cent, assign),
        }
        return spec, step, cpu_leg, None

    if c == "c4bin":
        # binary quantization of config 4's data (one bit per dimension,
        # x > 0) and the Hamming top-k scan (vsk_bin_search)
        from vectorstorekit_amd import BinaryDatabase, BinaryQuantizer
        n, d, nq, k = 10_000_000, 128, 1000, 100
        x, q = gen_flat(n, d, nq, False, dev)
        bq = BinaryQuantizer(ctx)
        xc, qc = bq.quantizeBatch(x), bq.quantizeBatch(q)
        del x
        db = BinaryDatabase(ctx, xc, d)
        dist = torch.empty(nq, k, dtype=torch.int32, device=dev)
        ids = torch.empty(nq, k, dtype=torch.int64, device=dev)

        def step():
            ctx.check(lib.vsk_bin_search(ctx.handle, db.handle, qc.data_ptr(), nq, k,
                                         dist.data_ptr(), ids.data_ptr()))

        def cpu_leg(target_s):
            from oracle import oracle as O
            xh, qh = xc.cpu().numpy(), qc.cpu().numpy()
            th = host_threads()
            qps, m, reps, el, (od, oi) = cpu_sample(
                lambda m: O.bin_search(qh[:m], xh, d, k, threads=th), nq, target_s, th)
            gd, gi = dist.cpu().numpy()[:m], ids.cpu().numpy()[:m]
            exact = {"queries": m, "ids_equal": bool((gi == oi).all()),
                     "distances_equal": bool((gd == od).all())}
            return ({"value": qps, "unit": "queries/s", "cores": th, "kind": "port",
                     "cpu": cpu_model(),
                     "sample": f"first {m} of {nq} queries against all {n} codes, {reps} "
                               f"pass(es) ({el:.1f} s)", "exact_oracle_check": exact},
                    id_agreement(gi, oi))

        spec = {
            "metric": "QPS @k=100, binary Hamming 10M x 128 bits",
            "workload": "bin-hamming-10Mx128-q1000-k100 (BASELINE config 4 data, binary codes)",
            "config": {"n": n, "d": d, "nq": nq, "k": k, "metric": "popcount(q xor x)"},
            "data": "synthetic: N(0,1) rows and queries (torch Philox seeds 1, 2), one bit "
                    "per dimension (x > 0)",
            "dtype": "u1 codes (int8 MFMA on 0/1 bytes)", "nq": nq, "n": n, "d": d, "words": 4,
            "kernels": [("bin_mfma_filter", "k_bin_mfma<2, 2, 8, FILTER> (int8 MFMA on bits "
                         "spread to bytes: H = |q| + |x| - 2 q.x)", "int8"),
                        ("bin_mfma_dense", "k_bin_mfma<2, 2, 8, DENSE>", "int8"),
                        ("bin_hamming_filter", "k_bin_scan<4, FILTER> (popcount)", "valu_bin"),
                        ("bin_hamming_dense", "k_bin_scan<4, DENSE> (popcount)", "valu_bin")],
            "keep": (db, xc, qc, dist, ids),
        }
        return spec, step, cpu_leg, None

    if c == "c3":
        n, d, ncent, nq, nprobe, k = 1_000_000, 128, 4096, 10_000, 32, 10
        x, q, cent = gen_mixture(n, d, ncent, nq, dev)
        idx = IVFIndex(ctx, IVFConfiguration(dimensions=d, numberOfCentroids=ncent,
                                             numberOfProbes=nprobe))
        idx.set_centroids(cent.cpu().numpy())
        idx.insert(x)
        dist = torch.empty(nq, k, device=dev)
        ids = torch.empty(nq, k, dtype=torch.int64, device=dev)

        def step():
            ctx.check(lib.vsk_ivf_search(ctx.handle, idx.handle, q.data_ptr(), nq, nprobe, k,
                                         L.METRIC_L2, dist.data_ptr(), ids.data_ptr()))

        qhost = q.cpu().numpy()
        hd, hi = np.empty((nq, k), np.float32), np.empty((nq, k), np.int64)

        def host_step():
            ctx.check(lib.vsk_ivf_search(ctx.handle, idx.handle, qhost.ctypes.data, nq, nprobe,
                                         k, L.METRIC_L2, hd.ctypes.data, hi.ctypes.data))

        def cpu_leg(target_s):
            from oracle import oracle as O
            xh, qh, ch = x.cpu().numpy(), qhost, idx.getCentroids()
            lists = idx.assign(x).cpu().numpy()
            rid = np.arange(n, dtype=np.int64)
            th = host_threads()
            qps, m, reps, el, (od, oi) = cpu_sample(
                lambda m: O.ivf_search(qh[:m], xh, rid, lists, ch, nprobe, k, threads=th),
                nq, target_s, th)
            gd, gi = dist.cpu().numpy(), ids.cpu().numpy()
            return ({"value": qps, "unit": "queries/s", "cores": th, "kind": "port",
                     "cpu": cpu_model(),
                     "sample": f"first {m} of {nq} queries, probe + scan of 32 lists "
                               f"(index built from the GPU's assignment; list build inside "
                               f"each oracle call), {reps} pass(es) ({el:.1f} s)",
                     "exact_oracle_check": exact_check(gd, gi, od, oi, m)},
                    id_agreement(gi[:m], oi))

        spec = {
            "metric": "QPS @k=10, IVF-Flat L2 1M x 128, nlist 4096, nprobe 32",
            "workload": "ivf-flat-l2-1Mx128-nlist4096-nprobe32-q10000-k10 (BASELINE config 3)",
            "config": {"n": n, "d": d, "nlist": ncent, "nprobe": nprobe, "nq": nq, "k": k,
                       "metric": "sqrt(sum (q-x)^2)"},
            "data": "synthetic: 4,096-Gaussian mixture, centres 2 N(0,I) (seed 3), "
                    "points centre + 0.5 N(0,I) (seeds 5, 1, 2), centroids centre + "
                    "0.1 N(0,I) (seed 4); torch Philox",
            "dtype": "f32", "nq": nq, "n": n, "d": d,
            "pairs_per_step": probed_pairs(idx, q, nprobe),
            "kernels": [("ivf_list_screen", "k_list_screen<4, false> (bf16 MFMA screen of the "
                                            "probed lists, one 32-bit word per pair)",
                         "words_hbm"),
                        ("ivf_list_scan", "k_list_scan<16>", "valu")],
            "keep": (idx, x, q, dist, ids),
        }
        return spec, step, cpu_leg, host_step

    if c in ("c3sq8", "c3pq"):
        # config 3's index with quantized lists: the same probing, the
        # probed lists scanned over SQ8 (per-dimension) or PQ M16x256 codes
        n, d, ncent, nq, nprobe, k = 1_000_000, 128, 4096, 10_000, 32, 10
        x, q, cent = gen_mixture(n, d, ncent, nq, dev)
        idx = IVFIndex(ctx, IVFConfiguration(dimensions=d, numberOfCentroids=ncent,
                                             numberOfProbes=nprobe))
        idx.set_centroids(cent.cpu().numpy())
        idx.insert(x)
        ids = torch.empty(nq, k, dtype=torch.int64, device=dev)
        M = 16
        if c == "c3sq8":
            sq = ScalarQuantizer(ctx, per_dim=True)
            sq.train(x)
            idx.encodeSQ8(sq)
            qc = sq.quantizeBatch(q)
            score = torch.empty(nq, k, dtype=torch.int32, device=dev)

            def step():
                ctx.check(lib.vsk_ivf_search_sq8(ctx.handle, idx.handle, q.data_ptr(),
                                                 qc.data_ptr(), nq, nprobe, k,
                                                 score.data_ptr(), ids.data_ptr()))
        else:
            g = torch.Generator(device="cpu").manual_seed(6)
            pick = torch.randperm(n, generator=g)[:256].to(dev)
            cb = x[pick].reshape(256, M, d // M).permute(1, 0, 2).contiguous().cpu().numpy()
            pq = ProductQuantizer(ctx, cb)
            idx.encodePQ(pq)
            dist = torch.empty(nq, k, device=dev)

            def step():
                ctx.check(lib.vsk_ivf_search_pq(ctx.handle, idx.handle, pq.handle,
                                                q.data_ptr(), nq, nprobe, k, dist.data_ptr(),
                                                ids.data_ptr()))

        def cpu_leg(target_s):
            from oracle import oracle as O
            xh, qh, ch = x.cpu().numpy(), q.cpu().numpy(), idx.getCentroids()
            lists = idx.assign(x).cpu().numpy()
            rid = np.arange(n, dtype=np.int64)
            if c == "c3sq8":
                codes = O.sq8_encode(xh, sq.scale, sq.offset)
                qch = qc.cpu().numpy()
                run = lambda m: O.ivf_sq8_search(qh[:m], qch[:m], codes, rid, lists, ch,
                                                 nprobe, k)
            else:
                codes = O.pq_encode(xh, cb, threads=host_threads())
                run = lambda m: O.ivf_pq_search(qh[:m], cb, codes, rid, lists, ch, nprobe, k)
            qps, m, reps, el, (od, oi) = cpu_sample(run, nq, target_s, 1)
            return ({"value": qps, "unit": "queries/s", "cores": 1, "kind": "port",
                     "cpu": cpu_model(),
                     "sample": f"first {m} of {nq} queries, probe + scan of 32 lists' codes "
                               f"(numpy over the oracle's probe; codes encoded outside the "
                               f"timing), {reps} pass(es) ({el:.1f} s)"},
                    id_agreement(ids.cpu().numpy()[:m], oi))

        # the quantized index keeps its codes only (vsk_ivf_drop_rows): the
        # searches read nothing else
        _, with_rows = idx.storage()
        idx.dropRows()
        _, codes_only = idx.storage()
        sq8 = c == "c3sq8"
        spec = {
            "metric": ("QPS @k=10, IVF-SQ8 (per-dim int8) 1M x 128, nlist 4096, nprobe 32" if sq8
                       else "QPS @k=10, IVF-PQ M16x256 1M x 128, nlist 4096, nprobe 32"),
            "workload": (f"ivf-{'sq8' if sq8 else 'pq16'}-1Mx128-nlist4096-nprobe32-q10000-k10 "
                         "(BASELINE config 3's index, quantized lists)"),
            "config": {"n": n, "d": d, "nlist": ncent, "nprobe": nprobe, "nq": nq, "k": k,
                       "metric": ("score sum qcode*code (descending)" if sq8 else
                                  "sqrt of the ADC sum of LUT[m][code_m]")},
            "data": "synthetic: config 3's mixture (as c3)"
                    + ("" if sq8 else "; codebooks: 256 random rows (seed 6) split in 16 "
                                      "segments"),
            "dtype": "i8 codes, i32 scores" if sq8 else "u8 codes, f32 LUT",
            "nq": nq, "n": n, "d": d, "M": M,
            "pairs_per_step": probed_pairs(idx, q, nprobe),
            "kernels": [("ivf_sq8_list_scan", "k_list_scan_sq8<16>", "valu_dot4")] if sq8
                       else [("ivf_pq_list_scan", "k_list_scan_pq_q (one workgroup per query)", "lds_pq")],
            "device_bytes": {"index_codes_only": codes_only, "index_with_fp32_rows": with_rows},
            "keep": (idx, x, q, ids, sq if sq8 else pq),
        }
        return spec, step, cpu_leg, None

    if c == "c4":
        n, d, nq, k = 10_000_000, 128, 1000, 100
        x, q = gen_flat(n, d, nq, False, dev)
        sq = ScalarQuantizer(ctx, per_dim=True)
        sq.train(x)
        codes = sq.quantizeBatch(x)
        del x
        qc = sq.quantizeBatch(q)
        db = SQ8Database(ctx, codes)
        score = torch.empty(nq, k, dtype=torch.int32, device=dev)
        ids = torch.empty(nq, k, dtype=torch.int64, device=dev)

        def step():
            ctx.check(lib.vsk_sq8_search(ctx.handle, db.handle, qc.data_ptr(), nq, k,
                                         score.data_ptr(), ids.data_ptr()))

        qhost = qc.cpu().numpy()
        hs, hi = np.empty((nq, k), np.int32), np.empty((nq, k), np.int64)

        def host_step():
            ctx.check(lib.vsk_sq8_search(ctx.handle, db.handle, qhost.ctypes.data, nq, k,
                                         hs.ctypes.data, hi.ctypes.data))

        def cpu_leg(target_s):
            from oracle import oracle as O
            ch, qh = codes.cpu().numpy(), qhost
            th = host_threads()
            qps, m, reps, el, (os_, oi) = cpu_sample(
                lambda m: O.sq8_search(qh[:m], ch, k, threads=th), nq, target_s, th)
            gs, gi = score.cpu().numpy(), ids.cpu().numpy()
            return ({"value": qps, "unit": "queries/s", "cores": th, "kind": "port",
                     "cpu": cpu_model(),
                     "sample": f"first {m} of {nq} queries against all {n} codes, "
                               f"{reps} pass(es) ({el:.1f} s)",
                     "exact_oracle_check": exact_check(gs, gi, os_, oi, m)},
                    id_agreement(gi[:m], oi))

        spec = {
            "metric": "QPS @k=100, int8 SQ dot scan 10M x 128",
            "workload": "sq8-dot-10Mx128-q1000-k100 (BASELINE config 4)",
            "config": {"n": n, "d": d, "nq": nq, "k": k,
                       "metric": "-sum code_q code_x (int32)", "quantiser": "per-dim min/max"},
            "data": "synthetic: N(0,1) rows and queries (torch Philox seeds 1, 2), "
                    "quantised per dimension",
            "dtype": "i8 (i32 accumulate)", "nq": nq, "n": n, "d": d,
            "kernels": [("sq8_mfma_filter", "k_sq8_pipe (int8 MFMA 16x16x64, filter test "
                                            "pipelined with the next block's MFMAs)", "int8"),
                        ("sq8_mfma_dense", "k_sq8_reg<DENSE> (int8 MFMA 16x16x64)", "int8")],
            "keep": (db, codes, qc, score, ids),
        }
        return spec, step, cpu_leg, host_step

    # c5 / c5lut
    n, d, nq, M, ksub, k_adc, k = 10_000_000, 128, 1000, 16, 256, 1000, 100
    x, q, _ = gen_mixture(n, d, 1024, nq, dev, jitter=False)
    pq = ProductQuantizer.train(ctx, x[:65536], M, ksub, iterations=8, seed=0)
    codes = pq.encode(x)
    pq.add(codes)
    db = VectorDatabase(ctx, x)
    dist = torch.empty(nq, k, device=dev)
    ids = torch.empty(nq, k, dtype=torch.int64, device=dev)
    l1 = L.METRIC_L1
    lut = c == "c5lut"
    sctx = ctx
    if lut:
        # codes only: a context without the bf16 screen (VSK_FLAT_KERNEL=
        # exact) scans the codes with the LDS tables, no decoded plane
        from vectorstorekit_amd import Context
        old = os.environ.get("VSK_FLAT_KERNEL")
        os.environ["VSK_FLAT_KERNEL"] = "exact"
        try:
            sctx = Context(0)
        finally:
            if old is None:
                del os.environ["VSK_FLAT_KERNEL"]
            else:
                os.environ["VSK_FLAT_KERNEL"] = old

    def step():
        sctx.check(lib.vsk_pq_search(sctx.handle, pq.handle, q.data_ptr(), nq, k_adc, k, l1,
                                     db.handle, dist.data_ptr(), ids.data_ptr()))

    qhost = q.cpu().numpy()
    hd, hi = np.empty((nq, k), np.float32), np.empty((nq, k), np.int64)

    def host_step():
        sctx.check(lib.vsk_pq_search(sctx.handle, pq.handle, qhost.ctypes.data, nq, k_adc, k,
                                     l1, db.handle, hd.ctypes.data, hi.ctypes.data))

    def cpu_leg(target_s):
        from oracle import oracle as O
        xh, qh, ch = x.cpu().numpy(), qhost, codes.cpu().numpy()
        th = host_threads()
        qps, m, reps, el, (od, oi) = cpu_sample(
            lambda m: O.pq_search(qh[:m], pq.codebooks, ch, k_adc, k, x=xh, rerank_metric=l1,
                                  threads=th), nq, target_s, th)
        gd, gi = dist.cpu().numpy(), ids.cpu().numpy()
        return ({"value": qps, "unit": "queries/s", "cores": th, "kind": "port",
                 "cpu": cpu_model(),
                 "sample": f"first {m} of {nq} queries: ADC over all {n} codes, top-1000, "
                           f"L1 re-rank, {reps} pass(es) ({el:.1f} s)",
                 "exact_oracle_check": exact_check(gd, gi, od, oi, m)},
                id_agreement(gi[:m], oi))

    code_bytes = n * M
    plane_bytes = 0 if lut else n * ((d + 63) // 64 * 64) * 2
    spec = {
        "metric": "QPS @k=100, PQ M16x256 ADC 10M x 128, top-1000 L1 re-rank",
        "workload": ("pq-adc-10Mx128-m16-q1000-kadc1000-l1rerank-k100 (BASELINE config 5)"
                     if not lut else
                     "pq-adc-codes-only-10Mx128-m16-q1000-kadc1000-l1rerank-k100 (BASELINE "
                     "config 5, LUT scan over the codes, no decoded plane)"),
        "ctx": sctx,
        "device_bytes": {"codes": code_bytes, "decoded_bf16_plane": plane_bytes,
                         "note": "the search's index memory besides the fp32 rows the "
                                 "re-rank reads" + ("" if lut else
                                 "; the screen's decoded plane is 16x the codes")},
        "config": {"n": n, "d": d, "M": M, "ksub": ksub, "nq": nq, "k_adc": k_adc, "k": k,
                   "metric": "ADC sum of LUT[m][code_m]; re-rank sum |q-x|"},
        "data": "synthetic: 1,024-Gaussian mixture, centres 2 N(0,I) (seed 3), points "
                "centre + 0.5 N(0,I) (seeds 5, 1, 2); codebooks: 8 Lloyd iterations "
                "per segment on the first 65,536 rows (GPU assignment)",
        "dtype": "u8 codes, f32 LUT", "nq": nq, "n": n, "d": d, "M": M,
        # filtered chunks: the bf16 screen over the decoded rows (one bf16
        # product per pair), then the survivors' exact ADC sums; the dense
        # first chunk: the LUT scan
        "kernels": ([("flat_screen_filter", "k_flat_screen<FILTER> over the decoded PQ rows",
                      "mfma_bf16")] if not lut else []) +
                   [("pq_adc_filter", "k_pq_adc16<FILTER> (8 queries per workgroup)", "lds_pq"),
                    ("pq_adc_dense", "k_pq_adc16<DENSE> (8 queries per workgroup)", "lds_pq")],
        "keep": (pq, db, x, q, codes, dist, ids, sctx),
    }
    return spec, step, cpu_leg, host_step


# ----------------------------------------------------------------- roofline

def with_measured_peak(r, kind):
    """Adds the re-measured ceiling of the roofline's own unit, if one was
    measured for it (bf16 and int8 matrix cores, HBM copy bandwidth)."""
    if r is None or not MEASURED_PEAKS:
        return r
    m = None
    if kind == "mfma_bf16":
        m = MEASURED_PEAKS["bf16_tflops"]
    elif kind == "mfma":
        m = MEASURED_PEAKS["bf16_tflops"] / 3
    elif kind == "int8":
        m = MEASURED_PEAKS["int8_tops"]
    elif r.get("bound") == "hbm":
        # the copy rate: these kernels both read and write
        m = MEASURED_PEAKS["hbm_gbs"]
    if m:
        r["measured_peak"] = round(m, 1)
        r["frac_of_measured_peak"] = round(r["achieved"] / m, 4)
    return r


def roofline(spec, stats, full=None):
    """Dominant kernel's roofline from the library's event timers: its
    launches and time from ``stats`` (the timed steps, where only the
    candidate kernels carry timers), its work (pairs) per launch from
    ``full`` (further steps of the same workload under full profiling, which
    reads the device-side work counts back) when given."""
    d = spec["d"]
    best = None
    for key, label, kind in spec["kernels"]:
        if key in stats and stats[key][1] > 0:
            if best is None or stats[key][1] > stats[best[0]][1]:
                best = (key, label, kind)
    if best is None:
        return None
    key, label, kind = best
    launches, ms, pairs = stats[key]
    if full is not None and key in full and full[key][0]:
        pairs = full[key][2] / full[key][0] * launches
    sec = ms * 1e-3
    r = {"kernel": f"{key} ({label})", "launches": launches,
         "avg_launch_ms": round(ms / launches, 4) if launches else None,
         "pairs_per_launch": pairs / launches if launches else None}
    if kind in ("mfma", "mfma32", "mfma_bf16"):
        flop = 2.0 * d * pairs
        peak = {"mfma": PEAK_BF16_MFMA_TFLOPS / 3, "mfma32": PEAK_FP32_MFMA_TFLOPS,
                "mfma_bf16": PEAK_BF16_MFMA_TFLOPS}[kind]
        ach = flop / sec / 1e12
        r.update({"bound": "mfma", "achieved": round(ach, 2), "peak": round(peak, 1),
                  "unit": "TFLOP/s", "frac": round(ach / peak, 4),
                  "algorithmic": "2*d FLOP per (query, row) pair",
                  "peak_basis": {
                      "mfma": "bf16 dense MFMA 2500 TFLOP/s / 3 products per fp32 product",
                      "mfma32": "fp32 dense MFMA",
                      "mfma_bf16": "bf16 dense MFMA 2500 TFLOP/s (the screen: one bf16 "
                                   "product per pair; final distances are exact fp32 "
                                   "rescores)"}[kind],
                  "frac_of_fp32_mfma_peak": round(ach / PEAK_FP32_MFMA_TFLOPS, 4)})
    elif kind == "int8":
        ops = 2.0 * d * pairs
        ach = ops / sec / 1e12
        r.update({"bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_INT8_MFMA_TOPS,
                  "unit": "TOP/s", "frac": round(ach / PEAK_INT8_MFMA_TOPS, 4),
                  "algorithmic": "2*d int8 OP per (query, row) pair",
                  "peak_basis": "int8 dense MFMA 5.0 POP/s"})
    elif kind in ("valu", "valu_l2", "valu_dot"):
        # exact fp32 sums in dimension order, no fused multiply-add, no
        # packed fp32: (q - x)^2 is a subtract, a multiply and an add per
        # dimension, q.x a multiply and an add
        flop = (2.0 if kind == "valu_dot" else 3.0) * d * pairs
        ach = flop / sec / 1e12
        r.update({"bound": "valu", "achieved": round(ach, 2), "peak": PEAK_FP32_VALU_TFLOPS,
                  "unit": "TFLOP/s", "frac": round(ach / PEAK_FP32_VALU_TFLOPS, 4),
                  "algorithmic": ("2*d" if kind == "valu_dot" else "3*d")
                                 + " fp32 operations per (query, row) pair",
                  "peak_basis": "fp32 vector 157.3 TFLOP/s (packed FMA); with one non-packed, "
                                "non-fused operation per lane per cycle the issue ceiling is "
                                f"{PEAK_FP32_VALU_ISSUE_TOPS} T operations/s",
                  "frac_of_issue_ceiling": round(ach / PEAK_FP32_VALU_ISSUE_TOPS, 4)})
        if kind == "valu":
            # the probed-list-bytes basis: above the HBM peak, because a list
            # row is read once for all the queries of a group that probe it
            r["list_bytes_basis"] = {"bytes_per_pair": 4 * d,
                                     "achieved_GBps": round(4.0 * d * pairs / sec / 1e9, 1),
                                     "frac_of_hbm": round(4.0 * d * pairs / sec / 1e9
                                                          / PEAK_HBM_GBPS, 4)}
    elif kind == "words_hbm":
        # the screened list scan reads the probed lists' bf16 plane
        # (2 * roundup(d, 64) bytes a row): at this configuration's nq x
        # nprobe every list is probed, so the plane is read once whole per
        # launch (a list read by two 128-query groups counts once).  That
        # is the algorithmic traffic.  The 32-bit screened distances it
        # writes (by default only the candidates under each query's bound,
        # compacted; with VSK_IVF_COMPACT=0 one per (query, candidate)
        # pair) are an intermediate the tail reads back: the every-pair
        # figure is reported beside it as an upper bound, not counted.  Its
        # bf16 products are 2*d FLOP a pair.
        ldb = (d + 63) // 64 * 64
        plane = 2.0 * ldb * spec["n"] * launches
        by = plane
        ach = by / sec / 1e9
        r.update({"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBPS,
                  "unit": "GB/s", "frac": round(ach / PEAK_HBM_GBPS, 4),
                  "algorithmic": "the bf16 plane of the probed lists read once per launch "
                                 "(2*roundup(d,64) bytes per row, every row at this nprobe)",
                  "with_every_word": {"bytes_per_launch": (4.0 * pairs + plane) / launches,
                                      "achieved_GBps": round((4.0 * pairs + plane) / sec / 1e9,
                                                             1),
                                      "note": "plus a 4-byte screened word per (query, "
                                              "candidate) pair, the most the scan writes (by "
                                              "default it writes only the candidates under "
                                              "each query's bound)"},
                  "bf16_mfma_TFLOPs": round(2.0 * d * pairs / sec / 1e12, 2)})
    elif kind == "kpp":
        # per pick every row's distance to the new centroid: 4*d bytes read
        # per (row, pick) pair at least (the rows stream from HBM)
        by = 4.0 * d * pairs
        ach = by / sec / 1e9
        r.update({"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBPS,
                  "unit": "GB/s", "frac": round(ach / PEAK_HBM_GBPS, 4),
                  "algorithmic": "4*d bytes per (row, pick): every row read once per new "
                                 "centroid"})
    elif kind == "valu_bin":
        # one v_xor_b32 and one v_bcnt_u32_b32 per 32-bit word per pair
        ops = 2.0 * spec["words"] * pairs
        ach = ops / sec / 1e12
        r.update({"bound": "valu", "achieved": round(ach, 2),
                  "peak": PEAK_FP32_VALU_ISSUE_TOPS, "unit": "TOP/s",
                  "frac": round(ach / PEAK_FP32_VALU_ISSUE_TOPS, 4),
                  "algorithmic": "2 integer operations (xor, popcount-add) per 32-bit code "
                                 "word per (query, row) pair",
                  "peak_basis": "one 32-bit VALU operation per lane per cycle: 256 CUs x "
                                f"4 SIMDs x 16 lanes x 2.4 GHz = {PEAK_FP32_VALU_ISSUE_TOPS} "
                                "T operations/s",
                  "code_bytes_basis": {"bytes_per_pair": 4 * spec["words"],
                                       "hbm_bytes_per_launch_min": 4.0 * spec["words"]
                                       * spec["n"]}})
    elif kind == "hbm":
        by = 4.0 * d * pairs
        ach = by / sec / 1e9
        r.update({"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBPS,
                  "unit": "GB/s", "frac": round(ach / PEAK_HBM_GBPS, 4),
                  "algorithmic": "4*d bytes per (query, probed row) pair: every probed "
                                 "list row read once per query"})
    elif kind == "valu_dot4":
        # v_dot4_i32_i8: four int8 products and their sum per lane per op
        ops = 2.0 * d * pairs
        ach = ops / sec / 1e12
        peak = PEAK_FP32_VALU_ISSUE_TOPS * 8
        r.update({"bound": "valu", "achieved": round(ach, 2), "peak": round(peak, 1),
                  "unit": "TOP/s", "frac": round(ach / peak, 4),
                  "algorithmic": "2*d int8 OP per (query, row) pair",
                  "peak_basis": "v_dot4_i32_i8 at one op per lane-cycle: 8 OP x "
                                f"{PEAK_FP32_VALU_ISSUE_TOPS} T lane-cycles/s"})
    elif kind == "lds_pq":
        # the tables are read from LDS, one 4-byte lookup per (query, code
        # byte); the code stream itself is shared by the 8 queries of a
        # workgroup, so the per-query code bytes exceed the HBM peak
        M = spec["M"]
        look = 1.0 * M * pairs / sec
        ach = 4.0 * look / 1e9
        peak = 4.0 * PEAK_LDS_LOOKUPS / 1e9
        r.update({"bound": "lds", "achieved": round(ach, 1), "peak": round(peak, 1),
                  "unit": "GB/s", "frac": round(ach / peak, 4),
                  "algorithmic": "M table lookups (4 bytes each, from LDS) per (query, row) "
                                 "pair",
                  "peak_basis": "64 four-byte LDS banks per CU x 256 CUs x 2.4 GHz (random "
                                "8-bit codes make bank conflicts; the conflict-free rate is "
                                "the ceiling)",
                  "lds_lookups_per_s": look,
                  "code_bytes_basis": {"bytes_per_pair": M,
                                       "achieved_GBps": round(M * pairs / sec / 1e9, 1),
                                       "frac_of_hbm": round(M * pairs / sec / 1e9
                                                            / PEAK_HBM_GBPS, 4)}})
    else:  # hbm_pq
        M = spec["M"]
        by = 1.0 * M * pairs
        ach = by / sec / 1e9
        r.update({"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBPS,
                  "unit": "GB/s", "frac": round(ach / PEAK_HBM_GBPS, 4),
                  "algorithmic": "M code bytes per (query, row) pair: all codes read "
                                 "once per query",
                  "lds_lookups_per_s": M * pairs / sec,
                  # one LUT lookup per code byte, each a 4-byte LDS read: 64 banks
                  # per CU at 2.4 GHz bound the conflict-free rate
                  "lds_lookup_peak_per_s": PEAK_LDS_LOOKUPS,
                  "lds_lookup_frac": round(M * pairs / sec / PEAK_LDS_LOOKUPS, 4)})
    r["traffic"], r["traffic_source"] = traffic_for(key, spec["workload"])
    return with_measured_peak(r, kind)


def traffic_for(kernel_key, workload):
    """HBM bytes per launch of this kernel on this workload, looked up in the
    committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary (not measured by this
    run), and where it came from; (None, None) when the summary has no entry."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            doc = json.load(f)
        rows = doc["entries"]
    except (OSError, ValueError, KeyError):
        return None, None
    tag = workload.split(" ")[0]
    for e in rows:
        if e.get("kernel") == kernel_key and e.get("workload") == tag:
            src = ("profiles/hbm_traffic.json: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes "
                   f"at commit {e.get('commit', doc.get('commit', 'unrecorded'))}, scaled by "
                   "the plain-copy calibration; a lookup, not a counter of this run")
            return e.get("traffic_bytes_per_launch"), src
    return None, None


# --------------------------------------------------------------------- main

def measure(c, a, ctx, dev):
    """One configuration: build, W warm-up steps, K timed steps with inputs
    and outputs in HBM (the value), then the host-buffer timing and the CPU
    baseline.  Returns the JSON object of that configuration."""
    import torch

    t0 = time.perf_counter()
    spec, step, cpu_leg, host_step = setup(c, a, ctx, dev)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    progress(f"{c}: setup {build_s:.1f} s")

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    # (a workload may run on a context of its own)
    ctx = spec.get("ctx", ctx)
    # the timed steps carry HIP-event timers on the roofline's candidate
    # kernels only (two events a launch, no work counts read back)
    ctx.profile_only([key for key, _, _ in spec["kernels"]])
    ctx.profile(True)
    ctx.profile_reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        step()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    stats = ctx.profile_stats()
    progress(f"{c}: {a.steps} steps in {el * 1e3:.1f} ms")
    # the per-kernel breakdown and the work counts: further steps with every
    # kernel timed (not part of the value)
    ctx.profile_only(None)
    ctx.profile_reset()
    breakdown_steps = max(1, min(a.steps, 5))
    for _ in range(breakdown_steps):
        step()
    torch.cuda.synchronize()
    full = ctx.profile_stats()
    ctx.profile(False)

    nq, n = spec["nq"], spec["n"]
    qps = spec.get("units_per_step", nq) * a.steps / el
    out = {
        "metric": spec["metric"],
        "value": round(qps, 1),
        "unit": spec.get("unit", "queries/s"),
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(el * 1e3 / a.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": spec["dtype"],
        "data": spec["data"],
        "config": dict({"workload": spec["workload"]}, **spec["config"]),
        "distances_per_s": spec.get("pairs_per_step", nq * n) * a.steps / el,
        "roofline": roofline(spec, stats, full),
        "device_bytes": spec.get("device_bytes"),
        "measured_peaks": {k: round(v, 1) for k, v in MEASURED_PEAKS.items()} or None,
        "setup_s": round(build_s, 2),
        "kernels_steps": breakdown_steps,
        "kernels": {k: {"launches": v[0], "ms_total": round(v[1], 3), "pairs": v[2]}
                    for k, v in full.items()},
    }
    if host_step is not None and not a.no_host_io:
        # queries read from and results written to pageable host memory:
        # the library stages them through device buffers (PCIe both ways)
        host_step()
        torch.cuda.synchronize()
        reps = max(1, min(a.steps, 10))
        t0 = time.perf_counter()
        for _ in range(reps):
            host_step()
        torch.cuda.synchronize()
        hel = time.perf_counter() - t0
        out["host_io_inclusive"] = {
            "value": round(spec.get("units_per_step", nq) * reps / hel, 1),
            "unit": out["unit"], "steps": reps, "ms_per_step": round(hel * 1e3 / reps, 4),
            "note": "same call with host query and result buffers (H2D + D2H inside the "
                    "timed region); not the value basis"}
    if not a.no_cpu:
        base, agree = cpu_leg(a.cpu_seconds)
        out["cpu_baseline"] = base
        out["ids_agreement_vs_cpu"] = round(agree, 5)
        progress(f"{c}: cpu baseline {base['value']:.1f} {base['unit']}")
    else:
        out["cpu_baseline"] = None
    del spec, step, cpu_leg, host_step
    return out


def main():
    a = parse()
    if a.copy_calibration:
        copy_calibration(a.copy_calibration)
        return
    if a.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; multi-GPU sharding "
                          "is design-only (rows split across GPUs, one merge of k results)",
                          "n_gpus": a.gpus}))
        sys.exit(2)
    import gc

    import torch

    from vectorstorekit_amd import Context

    dev = torch.device("cuda:0")
    ctx = Context(0)
    try:
        MEASURED_PEAKS.update(ctx.measure_peaks())
        progress("measured peaks: " + ", ".join(f"{k} {v:.0f}" for k, v in MEASURED_PEAKS.items()))
    except Exception as e:  # the rooflines then carry the datasheet fractions only
        progress(f"peak measurement failed: {e}")
    if a.config != "all":
        out = measure(a.config, a, ctx, dev)
    else:
        # the headline (config 2) at the top level, the other BASELINE
        # configs under "configs", each measured the same way
        out = None
        others = {}
        for c in BASELINE_CONFIGS + EXTRA_CONFIGS:
            r = measure(c, a, ctx, dev)
            gc.collect()
            torch.cuda.empty_cache()
            if out is None:
                out = r
            else:
                others[c] = r
        out["configs"] = others
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()

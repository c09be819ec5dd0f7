"""Benchmark of the search hot path on one MI355X.

Workload: flat cosine search, 1,000,000 x 768 fp32 rows
(i.i.d. N(0,1), each L2-normalised), 10,000 queries drawn the same way,
k = 100, distance 1 - q.x.  One step = one vsk_search_flat call over all
10,000 queries with the database and the queries already in HBM.

Prints one JSON line: QPS (value), the roofline of the dominant kernel
(the fused scan: algorithmic FLOP 2*d per (query, row) pair of a launch over
its HIP-event time), and a CPU baseline (the oracle's flat search on this host's
cores over the first queries of the same workload).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32_MFMA_TFLOPS = 157.3  # MI355X dense fp32 matrix, datasheet
PEAK_BF16_MFMA_TFLOPS = 2500.0  # MI355X dense bf16 matrix, datasheet
PEAK_HBM_GBPS = 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=5)
    p.add_argument("--warmup", type=int, default=1)
    p.add_argument("--n", type=int, default=1_000_000)
    p.add_argument("--d", type=int, default=768)
    p.add_argument("--nq", type=int, default=10_000)
    p.add_argument("--k", type=int, default=100)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--cpu-seconds", type=float, default=15.0,
                   help="target length of the CPU baseline sample")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="only run a plain device copy of MIB MiB 3 times (the "
                        "reference kernel for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return p.parse_args()


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


def cpu_baseline(x_host, q_host, k, gi, metric_code, target_s):
    """Time the oracle's flat search (16-accumulator variant, all host
    threads) on the first queries of the workload; also returns the recall
    of the GPU's ids against the exact CPU answer on those queries."""
    import numpy as np

    from oracle import oracle as O

    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    t0 = time.perf_counter()
    O.search_flat(q_host[:threads], x_host, k, metric_code, threads=threads, fast=True)
    t1 = time.perf_counter()
    per_round = t1 - t0  # one query per thread
    rounds = max(1, int(target_s / max(per_round, 1e-3)))
    nsamp = min(len(q_host), rounds * threads)
    t0 = time.perf_counter()
    od, oi = O.search_flat(q_host[:nsamp], x_host, k, metric_code, threads=threads, fast=True)
    el = time.perf_counter() - t0
    hits = sum(len(set(a) & set(b)) for a, b in zip(gi[:nsamp].tolist(), oi.tolist()))
    return {
        "value": nsamp / el,
        "unit": "queries/s",
        "cores": threads,
        "kind": "port",
        "sample": f"first {nsamp} of {len(q_host)} queries against all "
                  f"{x_host.shape[0]} rows ({el:.1f} s)",
    }, hits / oi.size


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
    import numpy as np
    import torch

    from vectorstorekit_amd import Context, VectorDatabase
    from vectorstorekit_amd._lib import METRIC_COSINE_NORMALIZED

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    x = torch.randn(a.n, a.d, generator=g, device=dev)
    x /= x.norm(dim=1, keepdim=True)
    g.manual_seed(2)
    q = torch.randn(a.nq, a.d, generator=g, device=dev)
    q /= q.norm(dim=1, keepdim=True)
    torch.cuda.synchronize()

    ctx = Context(0)
    db = VectorDatabase(ctx, x)
    dist = torch.empty(a.nq, a.k, device=dev)
    ids = torch.empty(a.nq, a.k, dtype=torch.int64, device=dev)
    lib = ctx.lib

    def step():
        ctx.check(lib.vsk_search_flat(ctx.handle, db.handle, q.data_ptr(), a.nq, a.k,
                                      METRIC_COSINE_NORMALIZED, dist.data_ptr(),
                                      ids.data_ptr()))

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    ctx.profile(True)
    ctx.profile_reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        step()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    stats = ctx.profile_stats()
    ctx.profile(False)

    qps = a.nq * a.steps / el
    # dominant kernel: the filtered pass of the flat scan (rows after the
    # first, dense chunk).  Its algorithmic FLOP = 2 * d per (query, row)
    # pair the library counted for its launches.  The default kernel forms
    # each fp32 product from 3 bf16 MFMA products (hi/lo split), so its
    # ceiling in algorithmic FLOP/s is the bf16 dense peak / 3; the fp32
    # MFMA kernel's ceiling is the fp32 matrix peak.
    if "flat_bf16x3_filter" in stats:
        kname, peak = "flat_bf16x3_filter (k_flat_bf16x3<1,3>)", PEAK_BF16_MFMA_TFLOPS / 3
        launches, scan_ms, pairs = stats["flat_bf16x3_filter"]
    else:
        kname, peak = "flat_mfma_filter (k_flat_mfma<1,3>)", PEAK_FP32_MFMA_TFLOPS
        launches, scan_ms, pairs = stats.get("flat_mfma_filter", (0, 0.0, 0.0))
    flop = 2.0 * a.d * pairs
    achieved = flop / (scan_ms * 1e-3) / 1e12 if scan_ms > 0 else None
    kernels = {k: {"launches": v[0], "ms_total": round(v[1], 3), "pairs": v[2]}
               for k, v in stats.items()}

    out = {
        "metric": "QPS @k=100, 1M x 768 fp32 flat cosine",
        "value": round(qps, 1),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(el * 1e3 / a.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: N(0,1) rows and queries (torch Philox seeds 1, 2), L2-normalised",
        "config": {"workload": "flat-cosine-1Mx768-q10000-k100 (BASELINE config 2)",
                   "n": a.n, "d": a.d, "nq": a.nq, "k": a.k, "metric": "1 - q.x"},
        "distances_per_s": a.nq * a.n * a.steps / el,
        "roofline": {
            "bound": "mfma",
            "kernel": kname,
            "flop_per_launch": flop / launches if launches else None,
            "achieved": round(achieved, 2) if achieved else None,
            "peak": round(peak, 1),
            "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4) if achieved else None,
            "peak_basis": ("bf16 dense MFMA 2500 TFLOP/s / 3 products per fp32 product"
                           if peak != PEAK_FP32_MFMA_TFLOPS else "fp32 dense MFMA"),
            "frac_of_fp32_mfma_peak": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4)
            if achieved else None,
            "traffic": None,
            "launches": launches,
            "avg_launch_ms": round(scan_ms / launches, 4) if launches else None,
        },
        "kernels": kernels,
    }
    if not a.no_cpu:
        xh = x.cpu().numpy()
        qh = q.cpu().numpy()
        base, rec = cpu_baseline(xh, qh, a.k, ids.cpu().numpy(), METRIC_COSINE_NORMALIZED,
                                 a.cpu_seconds)
        out["cpu_baseline"] = base
        out["recall_vs_cpu"] = round(rec, 5)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)
    db.free()
    ctx.close()


if __name__ == "__main__":
    main()

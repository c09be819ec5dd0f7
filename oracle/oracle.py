"""numpy front end of the CPU oracle (oracle/libvsk_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as
the checker and by bench.py's cpu_baseline leg.  The product library never
imports it.  The C code restates the reference's CPU algorithms; each
function there cites the reference file:line it follows.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import c_float, c_int32, c_int64, c_uint64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libvsk_oracle.so")

L2SQ, L2, COSINE, COSINE_NORMALIZED, DOT, L1, HAMMING, COSINE_NOEPS = range(8)

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        P = c_void_p
        sig = {
            "vsko_l2sq": (c_float, [P, P, c_int32]),
            "vsko_dot": (c_float, [P, P, c_int32]),
            "vsko_l1": (c_float, [P, P, c_int32]),
            "vsko_distance": (c_float, [P, P, c_int32, c_int32]),
            "vsko_normalize": (None, [P, c_int64, c_int32, P]),
            "vsko_matmul": (None, [P, c_int64, c_int32, P, c_int64, P]),
            "vsko_hnsw_distance": (c_float, [P, P, c_int32, c_int32]),
            "vsko_hnsw_distances": (None, [P, c_int64, P, c_int32, P, P, c_int32, P]),
            "vsko_scalar_quantize_u8": (None, [P, c_int64, c_int32, c_int32, P, P, P]),
            "vsko_distances": (None, [P, c_int64, P, c_int64, c_int32, c_int32, P, c_int32]),
            "vsko_search_flat": (None, [P, c_int64, P, c_int64, c_int32, c_int32, c_int32, P, P,
                                        c_int32, c_int32]),
            "vsko_topk": (None, [P, c_int64, c_int32, P, P]),
            "vsko_flat_prepare": (c_void_p, [P, c_int64, c_int32, c_int32]),
            "vsko_flat_free": (None, [P]),
            "vsko_flat_search": (None, [P, P, c_int64, c_int32, c_int32, P, P, c_int32]),
            "vsko_ivf_assign": (None, [P, c_int64, P, c_int32, c_int32, P, c_int32]),
            "vsko_ivf_probe": (None, [P, c_int64, P, c_int32, c_int32, c_int32, P, c_int32]),
            "vsko_ivf_search": (None, [P, c_int64, P, P, P, c_int64, c_int32, P, c_int32,
                                       c_int32, c_int32, c_int32, P, P, c_int32]),
            "vsko_sq8_train": (None, [P, c_int64, c_int32, c_int32, P, P]),
            "vsko_sq8_encode": (None, [P, c_int64, c_int32, c_int32, P, P, P]),
            "vsko_sq8_decode": (None, [P, c_int64, c_int32, c_int32, P, P, P]),
            "vsko_sq8_dot": (c_int32, [P, P, c_int32]),
            "vsko_sq8_search": (None, [P, c_int64, P, c_int64, c_int32, c_int32, P, P, c_int32]),
            "vsko_pq_lut": (None, [P, P, c_int32, c_int32, c_int32, P]),
            "vsko_pq_encode": (None, [P, c_int64, P, c_int32, c_int32, c_int32, P, c_int32]),
            "vsko_pq_decode": (None, [P, c_int64, P, c_int32, c_int32, c_int32, P]),
            "vsko_pq_adc_sum": (c_float, [P, P, c_int32, c_int32]),
            "vsko_pq_adc_scan": (None, [P, P, c_int64, c_int32, c_int32, P]),
            "vsko_pq_search": (None, [P, c_int64, P, P, c_int64, c_int32, c_int32, c_int32,
                                      c_int32, c_int32, P, c_int32, P, P, c_int32]),
            "vsko_kmeans": (None, [P, c_int64, c_int32, c_int32, c_int32, c_uint64, P, c_int32]),
            "vsko_swift_bounded": (c_uint64, [P, c_uint64]),
            "vsko_kmeans_init_random": (None, [c_int64, c_int32, c_uint64, P]),
            "vsko_kmeans_init_plusplus": (c_int32, [P, c_int64, c_int32, c_int32, c_uint64, P,
                                                    c_int32]),
            "vsko_kmeans_cluster": (c_int32, [P, c_int64, c_int32, c_int32, c_int32, P, P,
                                              c_int32, c_float, c_uint64, P, P, P, P, P,
                                              c_int32]),
            "vsko_binary_encode": (None, [P, c_int64, c_int32, P]),
            "vsko_bin_hamming": (c_int32, [P, P, c_int32]),
            "vsko_bin_search": (None, [P, c_int64, P, c_int64, c_int32, c_int32, P, P, c_int32]),
            "vsko_num_threads": (c_int32, []),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _c(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a, a.ctypes.data


def num_threads() -> int:
    return int(lib().vsko_num_threads())


def distance(q, x, metric) -> float:
    q, qp = _c(q, np.float32)
    x, xp = _c(x, np.float32)
    return float(lib().vsko_distance(qp, xp, q.shape[-1], metric))


def scalar_quantize_u8(x, bits=8):
    """quantizeVectors(.scalar(bits:)) on the reference's CPU path: (codes
    n x d uint8, scale n, min n)."""
    x, xp = _c(x, np.float32)
    n, d = x.shape
    codes = np.empty((n, d), np.uint8)
    sc = np.empty(n, np.float32)
    mn = np.empty(n, np.float32)
    lib().vsko_scalar_quantize_u8(xp, n, d, bits, codes.ctypes.data, sc.ctypes.data,
                                  mn.ctypes.data)
    return codes, sc, mn


def hnsw_distance(q, x, metric) -> float:
    """HNSWIndex DistanceComputer.distance of two vectors."""
    q, qp = _c(q, np.float32)
    x, xp = _c(x, np.float32)
    return float(lib().vsko_hnsw_distance(qp, xp, q.shape[-1], metric))


def hnsw_distances(q, x, offsets, rows, metric):
    """Query i against rows[offsets[i]:offsets[i+1]] of x (CSR)."""
    q, qp = _c(q, np.float32)
    x, xp = _c(x, np.float32)
    off, op = _c(offsets, np.int64)
    r, rp = _c(rows, np.int32)
    out = np.empty(int(off[-1]), np.float32)
    lib().vsko_hnsw_distances(qp, q.shape[0], xp, x.shape[1], op, rp, metric, out.ctypes.data)
    return out


def normalize(x):
    """normalizeVectors: each row divided by sqrt(sum x^2) + 1e-8."""
    x, xp = _c(x, np.float32)
    out = np.empty_like(x)
    lib().vsko_normalize(xp, x.shape[0], x.shape[1], out.ctypes.data)
    return out


def matmul(a, b):
    """matrixMultiply: a (m x k) times b (k x n), each entry summed over k in
    order from 0, a product then a sum (MetalMatrixCompute.swift:791-806)."""
    a, ap = _c(a, np.float32)
    b, bp = _c(b, np.float32)
    assert a.ndim == 2 and b.ndim == 2 and a.shape[1] == b.shape[0]
    out = np.empty((a.shape[0], b.shape[1]), np.float32)
    lib().vsko_matmul(ap, a.shape[0], a.shape[1], bp, b.shape[1], out.ctypes.data)
    return out


def distances(q, x, metric, threads=0):
    q, qp = _c(q, np.float32)
    x, xp = _c(x, np.float32)
    out = np.empty((q.shape[0], x.shape[0]), np.float32)
    lib().vsko_distances(qp, q.shape[0], xp, x.shape[0], q.shape[1], metric,
                         out.ctypes.data, threads)
    return out


def search_flat(q, x, k, metric, threads=0, fast=False):
    q, qp = _c(q, np.float32)
    x, xp = _c(x, np.float32)
    nq = q.shape[0]
    od = np.empty((nq, k), np.float32)
    oi = np.empty((nq, k), np.int64)
    lib().vsko_search_flat(qp, nq, xp, x.shape[0], x.shape[1], k, metric, od.ctypes.data,
                           oi.ctypes.data, threads, 1 if fast else 0)
    return od, oi


class FlatDB:
    """A database prepared once for repeated exact searches (the CPU
    baseline's resident index); same results as search_flat."""

    def __init__(self, x, threads=0):
        self.x, xp = _c(x, np.float32)
        self.d = self.x.shape[1]
        self.h = lib().vsko_flat_prepare(xp, self.x.shape[0], self.d, threads)

    def search(self, q, k, metric, threads=0):
        q, qp = _c(q, np.float32)
        nq = q.shape[0]
        od = np.empty((nq, k), np.float32)
        oi = np.empty((nq, k), np.int64)
        lib().vsko_flat_search(self.h, qp, nq, k, metric, od.ctypes.data, oi.ctypes.data,
                               threads)
        return od, oi

    def __del__(self):
        if getattr(self, "h", None):
            lib().vsko_flat_free(self.h)
            self.h = None


def topk(dist, k):
    d, dp = _c(dist, np.float32)
    od = np.empty(k, np.float32)
    oi = np.empty(k, np.int64)
    lib().vsko_topk(dp, d.shape[0], k, od.ctypes.data, oi.ctypes.data)
    return od, oi


def ivf_assign(x, centroids, threads=0):
    x, xp = _c(x, np.float32)
    c, cp = _c(centroids, np.float32)
    out = np.empty(x.shape[0], np.int32)
    lib().vsko_ivf_assign(xp, x.shape[0], cp, c.shape[0], x.shape[1], out.ctypes.data, threads)
    return out


def ivf_probe(q, centroids, nprobe, threads=0):
    q, qp = _c(q, np.float32)
    c, cp = _c(centroids, np.float32)
    out = np.empty((q.shape[0], nprobe), np.int32)
    lib().vsko_ivf_probe(qp, q.shape[0], cp, c.shape[0], q.shape[1], nprobe, out.ctypes.data,
                         threads)
    return out


def ivf_search(q, x, ids, list_of, centroids, nprobe, k, threads=0, squared=False):
    q, qp = _c(q, np.float32)
    x, xp = _c(x, np.float32)
    ids, ip = _c(ids, np.int64)
    lo, lp = _c(list_of, np.int32)
    c, cp = _c(centroids, np.float32)
    nq = q.shape[0]
    od = np.empty((nq, k), np.float32)
    oi = np.empty((nq, k), np.int64)
    lib().vsko_ivf_search(qp, nq, xp, ip, lp, x.shape[0], x.shape[1], cp, c.shape[0], nprobe, k,
                          1 if squared else 0, od.ctypes.data, oi.ctypes.data, threads)
    return od, oi


def sq8_train(x, per_dim=True):
    x, xp = _c(x, np.float32)
    d = x.shape[1]
    s = np.empty(d if per_dim else 1, np.float32)
    o = np.empty(d if per_dim else 1, np.float32)
    lib().vsko_sq8_train(xp, x.shape[0], d, 1 if per_dim else 0, s.ctypes.data, o.ctypes.data)
    return s, o


def sq8_encode(x, scale, offset):
    x, xp = _c(x, np.float32)
    s, sp = _c(scale, np.float32)
    o, op = _c(offset, np.float32)
    per_dim = 1 if s.shape[0] > 1 or x.shape[1] == 1 else 0
    out = np.empty(x.shape, np.int8)
    lib().vsko_sq8_encode(xp, x.shape[0], x.shape[1], per_dim, sp, op, out.ctypes.data)
    return out


def sq8_decode(codes, scale, offset):
    c, cp = _c(codes, np.int8)
    s, sp = _c(scale, np.float32)
    o, op = _c(offset, np.float32)
    per_dim = 1 if s.shape[0] > 1 or c.shape[1] == 1 else 0
    out = np.empty(c.shape, np.float32)
    lib().vsko_sq8_decode(cp, c.shape[0], c.shape[1], per_dim, sp, op, out.ctypes.data)
    return out


def sq8_search(qcodes, codes, k, threads=0):
    q, qp = _c(qcodes, np.int8)
    c, cp = _c(codes, np.int8)
    nq = q.shape[0]
    os_ = np.empty((nq, k), np.int32)
    oi = np.empty((nq, k), np.int64)
    lib().vsko_sq8_search(qp, nq, cp, c.shape[0], c.shape[1], k, os_.ctypes.data,
                          oi.ctypes.data, threads)
    return os_, oi


def pq_lut(q, codebooks):
    q, qp = _c(q, np.float32)
    cb, cbp = _c(codebooks, np.float32)
    M, ksub, dsub = cb.shape
    out = np.empty((M, ksub), np.float32)
    lib().vsko_pq_lut(qp, cbp, M, ksub, dsub, out.ctypes.data)
    return out


def pq_encode(x, codebooks, threads=0):
    x, xp = _c(x, np.float32)
    cb, cbp = _c(codebooks, np.float32)
    M, ksub, dsub = cb.shape
    out = np.empty((x.shape[0], M), np.uint8)
    lib().vsko_pq_encode(xp, x.shape[0], cbp, M, ksub, dsub, out.ctypes.data, threads)
    return out


def pq_decode(codes, codebooks):
    c, cp = _c(codes, np.uint8)
    cb, cbp = _c(codebooks, np.float32)
    M, ksub, dsub = cb.shape
    out = np.empty((c.shape[0], M * dsub), np.float32)
    lib().vsko_pq_decode(cp, c.shape[0], cbp, M, ksub, dsub, out.ctypes.data)
    return out


def pq_adc_scan(lut, codes):
    l, lp = _c(lut, np.float32)
    c, cp = _c(codes, np.uint8)
    out = np.empty(c.shape[0], np.float32)
    lib().vsko_pq_adc_scan(lp, cp, c.shape[0], c.shape[1], l.shape[1], out.ctypes.data)
    return out


def pq_search(q, codebooks, codes, k_adc, k, x=None, rerank_metric=-1, threads=0):
    q, qp = _c(q, np.float32)
    cb, cbp = _c(codebooks, np.float32)
    c, cp = _c(codes, np.uint8)
    M, ksub, dsub = cb.shape
    xp = 0
    if x is not None:
        x, xp = _c(x, np.float32)
    nq = q.shape[0]
    od = np.empty((nq, k), np.float32)
    oi = np.empty((nq, k), np.int64)
    lib().vsko_pq_search(qp, nq, cbp, cp, c.shape[0], M, ksub, dsub, k_adc, k,
                         xp if x is not None else None, rerank_metric, od.ctypes.data,
                         oi.ctypes.data, threads)
    return od, oi


def kmeans(x, k, iters=10, seed=0, threads=0):
    x, xp = _c(x, np.float32)
    out = np.empty((k, x.shape[1]), np.float32)
    lib().vsko_kmeans(xp, x.shape[0], x.shape[1], k, iters, seed, out.ctypes.data, threads)
    return out


def swift_bounded(state: int, bound: int):
    """Int.random(in: 0..<bound) on SeedableRNG(state): (value, new state)."""
    st = c_uint64(state)
    v = lib().vsko_swift_bounded(ctypes.byref(st), bound)
    return int(v), int(st.value)


def kmeans_init_random(n, k, seed):
    rows = np.empty(k, np.int64)
    lib().vsko_kmeans_init_random(n, k, seed, rows.ctypes.data)
    return rows


def kmeans_init_plusplus(x, k, seed, threads=0):
    """k-means++ starting rows, or None on degenerate data."""
    x, xp = _c(x, np.float32)
    rows = np.empty(k, np.int64)
    rc = lib().vsko_kmeans_init_plusplus(xp, x.shape[0], x.shape[1], k, seed, rows.ctypes.data,
                                         threads)
    return None if rc != 0 else rows


INIT_METHODS = {"random": 0, "custom": 1, "kMeansPlusPlus": 2}


def kmeans_cluster(x, k, init_method="random", init=None, weights=None, max_iter=100,
                   tol=1e-4, seed=0, threads=0):
    """KMeansClustering.cluster restated: (centroids, assignments, iterations,
    converged, inertia); raises ValueError on degenerate data."""
    x, xp = _c(x, np.float32)
    n, d = x.shape
    ip = wp = None
    if init is not None:
        init, ip = _c(init, np.float32)
    if weights is not None:
        weights, wp = _c(weights, np.float32)
    cent = np.empty((k, d), np.float32)
    assign = np.empty(n, np.int32)
    it = c_int32(0)
    conv = c_int32(0)
    inertia = c_float(0)
    rc = lib().vsko_kmeans_cluster(xp, n, d, k, INIT_METHODS[init_method], ip, wp, max_iter,
                                   tol, seed, cent.ctypes.data, assign.ctypes.data,
                                   ctypes.byref(it), ctypes.byref(conv), ctypes.byref(inertia),
                                   threads)
    if rc != 0:
        raise ValueError("degenerate data")
    return cent, assign, int(it.value), bool(conv.value), np.float32(inertia.value)


def binary_encode(x):
    """AccelerateOptimizer.binaryQuantize: (n, ceil(d/8)) uint8."""
    x, xp = _c(x, np.float32)
    n, d = x.shape
    out = np.empty((n, (d + 7) // 8), np.uint8)
    lib().vsko_binary_encode(xp, n, d, out.ctypes.data)
    return out


def bin_search(qcodes, codes, d, k, threads=0):
    """top k by (Hamming distance, id): (int32 distances, int64 ids)."""
    q, qp = _c(qcodes, np.uint8)
    c, cp = _c(codes, np.uint8)
    nq = q.shape[0]
    od = np.empty((nq, k), np.int32)
    oi = np.empty((nq, k), np.int64)
    lib().vsko_bin_search(qp, nq, cp, c.shape[0], d, k, od.ctypes.data, oi.ctypes.data, threads)
    return od, oi


def _ivf_candidates(q, list_of, centroids, nprobe):
    """Per query: the candidate rows of IVFIndex.search (Indexes/
    IVFIndex.swift:149-202) in its concatenation order -- probed lists in
    probe order, each list's rows in insertion (row) order."""
    list_of = np.asarray(list_of)
    probes = ivf_probe(q, centroids, nprobe)
    members = {}
    out = []
    for pr in probes:
        rows = []
        for l in pr:
            if l < 0:
                continue
            if l not in members:
                members[l] = np.nonzero(list_of == l)[0]
            rows.append(members[l])
        out.append(np.concatenate(rows) if rows else np.zeros(0, np.int64))
    return out


def ivf_sq8_search(q, qcodes, codes, ids, list_of, centroids, nprobe, k):
    """IVF-SQ8: probe as ivf_search, score the candidates' codes with
    sq8 scores (int64 dot of int8 codes), stable order by descending
    score; (scores int32 [nq, k], ids) padded with INT32_MIN / -1."""
    qc = np.asarray(qcodes, np.int64)
    codes = np.asarray(codes, np.int64)
    ids = np.asarray(ids, np.int64)
    nq = qc.shape[0]
    os_ = np.full((nq, k), np.iinfo(np.int32).min, np.int32)
    oi = np.full((nq, k), -1, np.int64)
    for i, rows in enumerate(_ivf_candidates(q, list_of, centroids, nprobe)):
        sc = codes[rows] @ qc[i]
        order = np.argsort(-sc, kind="stable")[:k]
        os_[i, :len(order)] = sc[order]
        oi[i, :len(order)] = ids[rows[order]]
    return os_, oi


def ivf_pq_search(q, codebooks, codes, ids, list_of, centroids, nprobe, k):
    """IVF-PQ: probe as ivf_search, ADC sums of the candidates' codes
    (pq_adc_scan: fp32 in segment order), stable ascending order; returns
    (sqrt of the sum float32 [nq, k], ids) padded with +inf / -1."""
    q = np.ascontiguousarray(q, np.float32)
    codes = np.ascontiguousarray(codes, np.uint8)
    ids = np.asarray(ids, np.int64)
    nq = q.shape[0]
    od = np.full((nq, k), np.inf, np.float32)
    oi = np.full((nq, k), -1, np.int64)
    for i, rows in enumerate(_ivf_candidates(q, list_of, centroids, nprobe)):
        s = pq_adc_scan(pq_lut(q[i], codebooks), codes[rows])
        order = np.argsort(s, kind="stable")[:k]
        od[i, :len(order)] = np.sqrt(s[order])
        oi[i, :len(order)] = ids[rows[order]]
    return od, oi


def search_layer0(query, x, adjacency, entry, ef, metric, deleted=()):
    """HNSWIndex.searchLayer0 (Indexes/HNSWIndex.swift:1151-1212) restated
    in Python over adjacency lists, with DistanceComputer's distances
    (vsko_hnsw_distance).  The sorts are stable (Python's sort; Swift's
    sort is stable in its implementation, not by contract).  Returns the
    ef closest (distance, node) pairs ascending.  Small cases only."""
    deleted = set(deleted)
    d0 = hnsw_distance(query, x[entry], metric)
    visited = {entry}
    candidates = [(d0, entry)]
    w = [(d0, entry)]
    while candidates:
        candidates.sort(key=lambda t: t[0])
        cur = candidates.pop(0)
        if len(w) >= ef:
            w.sort(key=lambda t: t[0], reverse=True)
            if cur[0] > w[0][0]:
                break
        if cur[1] in deleted:
            continue
        for nb in adjacency[cur[1]]:
            if nb in visited:
                continue
            visited.add(nb)
            if nb in deleted:
                continue
            dist = hnsw_distance(query, x[nb], metric)
            if len(w) < ef:
                candidates.append((dist, nb))
                w.append((dist, nb))
            else:
                w.sort(key=lambda t: t[0], reverse=True)
                if dist < w[0][0]:
                    candidates.append((dist, nb))
                    w[0] = (dist, nb)
    w.sort(key=lambda t: t[0])
    return w

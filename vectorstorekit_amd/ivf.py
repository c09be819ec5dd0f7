"""``IVFIndex`` mirror over the C ABI (Indexes/IVFIndex.swift of
gifton/VectorStoreKit).

Reference surface kept: ``IVFConfiguration(dimensions, numberOfCentroids,
numberOfProbes)`` (Config/Indexes/IVFConfiguration.swift:8-92),
``train(on:)`` (:397-446), ``insert`` (:80-122), ``search(query, k,
strategy)`` (:124-202; ``"exact"`` probes every list, :551-554),
``getCentroids()`` (:483).  Search returns (distances, ids) arrays instead of
``SearchResult`` objects; distances are the reference's sqrt-L2.
"""
from __future__ import annotations

import ctypes
import json
import os
from dataclasses import dataclass, field

import numpy as np

from ._lib import VSKError, as_buffer, out_buffer, row_bitmap
from .clustering import ClusteringResult, KMeansClustering, KMeansClusteringConfiguration
from .engine import Context, metric_code


@dataclass
class IVFConfiguration:
    dimensions: int
    numberOfCentroids: int = 1024
    numberOfProbes: int = 10
    # the k-means that train(on:) runs (IVFConfiguration.clusteringConfig,
    # Config/Indexes/IVFConfiguration.swift:14,35; default .default)
    clusteringConfig: KMeansClusteringConfiguration = field(
        default_factory=KMeansClusteringConfiguration)

    def validate(self):
        if self.dimensions <= 0:
            raise VSKError(-2, "dimensions must be positive")
        if self.numberOfCentroids <= 0:
            raise VSKError(-2, "numberOfCentroids must be positive")
        if not 0 < self.numberOfProbes <= self.numberOfCentroids:
            raise VSKError(-2, "numberOfProbes must be in [1, numberOfCentroids]")


class IVFIndex:
    """IVF-Flat index resident on one GPU."""

    def __init__(self, ctx: Context, configuration: IVFConfiguration):
        configuration.validate()
        self.ctx = ctx
        self.configuration = configuration
        self.handle = None
        self._centroids = None
        self._sq8 = None  # the quantizers the stored codes were made with
        self._pq = None
        self.savedExtra = None

    @property
    def trained(self) -> bool:
        return self.handle is not None

    def set_centroids(self, centroids):
        """Adopt trained centroids (nlist, d)."""
        c = np.ascontiguousarray(centroids, np.float32)
        if c.shape != (self.configuration.numberOfCentroids, self.configuration.dimensions):
            raise VSKError(-4, f"centroids shape {c.shape}")
        self.free()
        h = ctypes.c_void_p()
        self.ctx.check(self.ctx.lib.vsk_ivf_create(self.ctx.handle, c.ctypes.data, c.shape[0],
                                                   c.shape[1], ctypes.byref(h)))
        self.handle = h
        self._centroids = c

    @classmethod
    def build(cls, ctx: Context, configuration: IVFConfiguration, centroids, vectors,
              ids=None) -> "IVFIndex":
        """Trained centroids plus the rows in one call (``vsk_ivf_build``):
        the same index as ``set_centroids`` followed by ``insert``."""
        configuration.validate()
        c = np.ascontiguousarray(centroids, np.float32)
        if c.shape != (configuration.numberOfCentroids, configuration.dimensions):
            raise VSKError(-4, f"centroids shape {c.shape}")
        n = int(vectors.shape[0])
        xp, xk = as_buffer(vectors, np.float32, (n, configuration.dimensions))
        ip, ik = (as_buffer(ids, np.int64, (n,)) if ids is not None else (None, None))
        h = ctypes.c_void_p()
        ctx.check(ctx.lib.vsk_ivf_build(ctx.handle, c.ctypes.data, c.shape[0], xp, ip, n,
                                        c.shape[1], ctypes.byref(h)))
        idx = cls(ctx, configuration)
        idx.handle = h
        idx._centroids = c
        return idx

    def train(self, on) -> ClusteringResult:
        """IVFIndex.train(on:) (Indexes/IVFIndex.swift:397-446, .kmeans): k-means
        with configuration.clusteringConfig on the GPU (vsk_kmeans), the
        centroids adopted, the lists emptied."""
        k = self.configuration.numberOfCentroids
        if on.shape[0] < k:
            raise VSKError(-2, f"insufficient training data: provided {on.shape[0]}, "
                           f"required {k}")
        res = KMeansClustering(self.ctx, self.configuration.clusteringConfig).cluster(on, k)
        cent = res.centroids
        self.set_centroids(cent.cpu().numpy() if hasattr(cent, "cpu") else cent)
        return res

    def getCentroids(self) -> np.ndarray:
        self._need()
        return self._centroids.copy()

    def _need(self):
        if self.handle is None:
            raise VSKError(-7, "IVF index must be trained before use")

    def assign(self, vectors) -> np.ndarray:
        self._need()
        n = int(vectors.shape[0])
        xp, xk = as_buffer(vectors, np.float32, (n, self.configuration.dimensions))
        op, out = out_buffer((n,), np.int32, vectors)
        self.ctx.check(self.ctx.lib.vsk_ivf_assign(self.ctx.handle, self.handle, xp, n, op))
        return out

    def insert(self, vectors, ids=None):
        self._need()
        n = int(vectors.shape[0])
        xp, xk = as_buffer(vectors, np.float32, (n, self.configuration.dimensions))
        ip, ik = (as_buffer(ids, np.int64, (n,)) if ids is not None else (None, None))
        self.ctx.check(self.ctx.lib.vsk_ivf_add(self.ctx.handle, self.handle, xp, ip, n))

    def probe(self, queries, nprobe=None) -> np.ndarray:
        self._need()
        nprobe = nprobe or self.configuration.numberOfProbes
        nq = int(queries.shape[0])
        qp, qk = as_buffer(queries, np.float32, (nq, self.configuration.dimensions))
        op, out = out_buffer((nq, nprobe), np.int32, queries)
        self.ctx.check(self.ctx.lib.vsk_ivf_probe(self.ctx.handle, self.handle, qp, nq,
                                                  nprobe, op))
        return out

    def search(self, queries, k: int, strategy: str = "approximate", nprobe=None,
               metric="euclidean", allow=None, allow_bits=None):
        """Top k by L2 over the probed lists; ``metric`` is "euclidean"
        (the reference's sqrt distance) or "euclideanSquared".  ``allow``
        (optional) filters the candidates before they are ranked, as
        IVFIndex.search's filter does (:161-176): a boolean array over the
        row ids, or the allowed ids (``vsk_ivf_search_filtered``)."""
        self._need()
        if strategy == "exact":
            nprobe = self.configuration.numberOfCentroids
        nprobe = nprobe or self.configuration.numberOfProbes
        q = queries
        if not hasattr(q, "shape") or len(q.shape) == 1:
            q = np.asarray(q, np.float32).reshape(1, -1)
        nq = int(q.shape[0])
        qp, qk = as_buffer(q, np.float32, (nq, self.configuration.dimensions))
        dp, dist = out_buffer((nq, k), np.float32, q)
        ip, ids = out_buffer((nq, k), np.int64, q)
        if allow is None:
            self.ctx.check(self.ctx.lib.vsk_ivf_search(self.ctx.handle, self.handle, qp, nq,
                                                       nprobe, k, metric_code(metric), dp, ip))
        else:
            bm = row_bitmap(allow, allow_bits)
            nbits = (int(np.asarray(allow).size) if np.asarray(allow).dtype == np.bool_
                     else int(bm.size * 32))
            self.ctx.check(self.ctx.lib.vsk_ivf_search_filtered(
                self.ctx.handle, self.handle, qp, nq, nprobe, k, metric_code(metric),
                bm.ctypes.data, nbits, dp, ip))
        return dist, ids

    def remove(self, ids) -> int:
        """IVFIndex.delete(id:) for device ids (:210-220): every stored row
        with one of these ids leaves its list (``vsk_ivf_remove``); returns
        how many rows were removed."""
        self._need()
        a = np.ascontiguousarray(np.asarray(ids, np.int64).reshape(-1))
        out = ctypes.c_int64(0)
        self.ctx.check(self.ctx.lib.vsk_ivf_remove(self.ctx.handle, self.handle, a.ctypes.data,
                                                   a.size, ctypes.byref(out)))
        return int(out.value)

    def listIds(self):
        """getVectorsFromList for every list (:487-490): (ids in list
        order, offsets[nlist + 1])."""
        self._need()
        off = np.empty(self.configuration.numberOfCentroids + 1, np.int64)
        self.ctx.check(self.ctx.lib.vsk_ivf_list_ids(self.ctx.handle, self.handle, None,
                                                     off.ctypes.data))
        ids = np.empty(int(off[-1]), np.int64)
        if ids.size:
            self.ctx.check(self.ctx.lib.vsk_ivf_list_ids(self.ctx.handle, self.handle,
                                                         ids.ctypes.data, None))
        return ids, off

    # ---- quantized lists (IVFConfiguration's declared quantization,
    # Config/Indexes/IVFConfiguration.swift:13,18-21, which IVFIndex leaves
    # unimplemented): codes of the stored rows, scored per probed list
    def encodeSQ8(self, quantizer):
        """Codes of every stored row with a trained ``ScalarQuantizer``;
        rows inserted later need another call before ``searchSQ8``."""
        self._need()
        quantizer._need()
        self.ctx.check(self.ctx.lib.vsk_ivf_encode_sq8(
            self.ctx.handle, self.handle, 1 if quantizer.per_dim else 0,
            quantizer.scale.ctypes.data, quantizer.offset.ctypes.data))
        self._sq8, self._pq = quantizer, None

    def encodePQ(self, pq):
        """PQ codes of every stored row with a trained ``ProductQuantizer``."""
        self._need()
        self.ctx.check(self.ctx.lib.vsk_ivf_encode_pq(self.ctx.handle, self.handle, pq.handle))
        self._sq8, self._pq = None, pq

    def dropRows(self):
        """Keep only the codes (``vsk_ivf_drop_rows``): the fp32 rows and
        their screen plane are freed.  ``searchSQ8`` / ``searchPQ`` answer as
        before; ``insert`` encodes new rows with the quantizer the codes were
        made with; ``search`` and ``encodeSQ8`` / ``encodePQ`` raise."""
        self._need()
        self.ctx.check(self.ctx.lib.vsk_ivf_drop_rows(self.ctx.handle, self.handle))

    @property
    def codesOnly(self) -> bool:
        return self.storage()[0]

    def storage(self):
        """(codes only, device bytes the index holds) (``vsk_ivf_storage``)."""
        self._need()
        co, nb = ctypes.c_int32(0), ctypes.c_int64(0)
        self.ctx.check(self.ctx.lib.vsk_ivf_storage(self.ctx.handle, self.handle,
                                                    ctypes.byref(co), ctypes.byref(nb)))
        return bool(co.value), int(nb.value)

    def _queries(self, queries):
        q = queries
        if not hasattr(q, "shape") or len(q.shape) == 1:
            q = np.asarray(q, np.float32).reshape(1, -1)
        return q, int(q.shape[0])

    def searchSQ8(self, queries, k: int, nprobe=None, strategy: str = "approximate"):
        """(scores [nq, k] int32 descending, ids): the int8 dot score of the
        query's codes with the probed lists' codes."""
        self._need()
        if strategy == "exact":
            nprobe = self.configuration.numberOfCentroids
        nprobe = nprobe or self.configuration.numberOfProbes
        if self._sq8 is None:
            raise VSKError(-7, "the index holds no SQ8 codes (encodeSQ8)")
        q, nq = self._queries(queries)
        qc = self._sq8.quantizeBatch(q)
        qp, qk = as_buffer(q, np.float32, (nq, self.configuration.dimensions))
        cp, ck = as_buffer(qc, np.int8, (nq, self.configuration.dimensions))
        sp, score = out_buffer((nq, k), np.int32, q)
        ip, ids = out_buffer((nq, k), np.int64, q)
        self.ctx.check(self.ctx.lib.vsk_ivf_search_sq8(self.ctx.handle, self.handle, qp, cp,
                                                       nq, nprobe, k, sp, ip))
        return score, ids

    def searchPQ(self, queries, k: int, nprobe=None, strategy: str = "approximate"):
        """(sqrt of the ADC sum [nq, k] ascending, ids) over the probed
        lists' PQ codes."""
        self._need()
        if strategy == "exact":
            nprobe = self.configuration.numberOfCentroids
        nprobe = nprobe or self.configuration.numberOfProbes
        if self._pq is None:
            raise VSKError(-7, "the index holds no PQ codes (encodePQ)")
        q, nq = self._queries(queries)
        qp, qk = as_buffer(q, np.float32, (nq, self.configuration.dimensions))
        dp, dist = out_buffer((nq, k), np.float32, q)
        ip, ids = out_buffer((nq, k), np.int64, q)
        self.ctx.check(self.ctx.lib.vsk_ivf_search_pq(self.ctx.handle, self.handle,
                                                      self._pq.handle, qp, nq, nprobe, k,
                                                      dp, ip))
        return dist, ids

    # ---- index file (the whole index; the reference's persistence keeps
    # only the configuration and centroids, Indexes/IVFIndex.swift:297-328)
    def save(self, path: str, extra=None):
        """The index, its codes and quantizer parameters, and this
        configuration (as JSON in the file's metadata) in one file.
        ``extra`` (JSON-serialisable, optional) is kept with it and comes
        back as ``savedExtra`` of the loaded index."""
        self._need()
        cfg = self.configuration
        meta = json.dumps({"extra": extra,
            "dimensions": cfg.dimensions, "numberOfCentroids": cfg.numberOfCentroids,
            "numberOfProbes": cfg.numberOfProbes,
            "clusteringConfig": {"maxIterations": cfg.clusteringConfig.maxIterations,
                                 "tolerance": cfg.clusteringConfig.tolerance,
                                 "initMethod": cfg.clusteringConfig.initMethod,
                                 "seed": cfg.clusteringConfig.seed}}).encode()
        self.ctx.check(self.ctx.lib.vsk_ivf_set_meta(self.ctx.handle, self.handle, meta,
                                                     len(meta)))
        self.ctx.check(self.ctx.lib.vsk_ivf_save(self.ctx.handle, self.handle,
                                                 os.fsencode(path)))

    @classmethod
    def load(cls, ctx: Context, path: str, sq8=None, pq=None) -> "IVFIndex":
        """An index written by ``save``, with its saved configuration.  SQ8
        codes come back with their quantizer (a passed ``sq8`` must equal
        it); PQ codes need the ``pq`` they were made with, which the library
        checks against the codebooks stored in the file at search time."""
        h = ctypes.c_void_p()
        ctx.check(ctx.lib.vsk_ivf_load(ctx.handle, os.fsencode(path), ctypes.byref(h)))
        try:
            nlist, d, kind = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
            total = ctypes.c_int64()
            ctx.check(ctx.lib.vsk_ivf_info(ctx.handle, h, ctypes.byref(nlist), ctypes.byref(d),
                                           ctypes.byref(total), ctypes.byref(kind)))
            n = ctypes.c_int64()
            ctx.check(ctx.lib.vsk_ivf_get_meta(ctx.handle, h, None, 0, ctypes.byref(n)))
            raw = ctypes.create_string_buffer(max(1, n.value))
            ctx.check(ctx.lib.vsk_ivf_get_meta(ctx.handle, h, raw, n.value, ctypes.byref(n)))
            meta = json.loads(raw.raw[:n.value].decode()) if n.value else {}
            cc = meta.get("clusteringConfig", {})
            cfg = IVFConfiguration(
                dimensions=d.value, numberOfCentroids=nlist.value,
                numberOfProbes=min(int(meta.get("numberOfProbes", 10)), nlist.value),
                clusteringConfig=KMeansClusteringConfiguration(
                    **{k: cc[k] for k in ("maxIterations", "tolerance", "initMethod", "seed")
                       if k in cc}))
            cent = np.empty((nlist.value, d.value), np.float32)
            ctx.check(ctx.lib.vsk_ivf_centroids(ctx.handle, h, cent.ctypes.data))
            sq = None
            if kind.value == 1:
                from .quantization import ScalarQuantizer

                pdim = ctypes.c_int32()
                ctx.check(ctx.lib.vsk_ivf_sq8_params(ctx.handle, h, ctypes.byref(pdim), None,
                                                     None))
                ns = d.value if pdim.value else 1
                sc, of = np.empty(ns, np.float32), np.empty(ns, np.float32)
                ctx.check(ctx.lib.vsk_ivf_sq8_params(ctx.handle, h, ctypes.byref(pdim),
                                                     sc.ctypes.data, of.ctypes.data))
                if sq8 is not None and (bool(sq8.per_dim) != bool(pdim.value)
                                        or not np.array_equal(sq8.scale, sc)
                                        or not np.array_equal(sq8.offset, of)):
                    raise VSKError(-4, "sq8 differs from the quantizer the codes were made "
                                   "with")
                sq = sq8 or ScalarQuantizer(ctx, per_dim=bool(pdim.value))
                sq.scale, sq.offset, sq.dimensions = sc, of, d.value
        except BaseException:
            ctx.lib.vsk_ivf_free(ctx.handle, h)
            raise
        idx = cls(ctx, cfg)
        idx.handle = h
        idx._centroids = cent
        idx.savedExtra = meta.get("extra")
        if kind.value == 1:
            idx._sq8 = sq
        elif kind.value == 2:
            idx._pq = pq
        return idx

    def list_sizes(self) -> np.ndarray:
        self._need()
        out = np.empty(self.configuration.numberOfCentroids, np.int64)
        self.ctx.check(self.ctx.lib.vsk_ivf_list_sizes(self.ctx.handle, self.handle,
                                                       out.ctypes.data))
        return out

    @property
    def count(self) -> int:
        return int(self.list_sizes().sum()) if self.trained else 0

    def free(self):
        if self.handle is not None:
            self.ctx.lib.vsk_ivf_free(self.ctx.handle, self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

"""Scalar (int8) and product quantizer mirrors over the C ABI.

* ``ScalarQuantizer`` -- Quantization/ScalarQuantizer.swift of
  gifton/VectorStoreKit: ``train`` (statistics + parameters, :389-451),
  ``quantizeBatch`` (:129-164 / quantizeToInt8 :251-270), ``dequantize``
  (:568-580, computed on the host: (code - offset) / scale), plus
  ``SQ8Database.search`` -- the int8 scan (no reference counterpart; ranks by
  the exact int32 dot of codes).
* ``ProductQuantizer`` -- Quantization/ProductQuantizer.swift:
  ``encode`` (:68-112), ``precomputeDistanceTables`` (:209-233), ``add``
  (resident codes), ``search`` (ADC scan over every code, optional exact
  re-rank).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import VSKError, as_buffer, out_buffer
from .engine import Context, VectorDatabase, metric_code


class ScalarQuantizer:
    """int8 scalar quantizer; ``per_dim`` False is the reference's global
    min/max, True the per-dimension variant."""

    def __init__(self, ctx: Context, per_dim: bool = True):
        self.ctx = ctx
        self.per_dim = per_dim
        self.scale = None
        self.offset = None

    def train(self, vectors):
        n, d = int(vectors.shape[0]), int(vectors.shape[1])
        xp, xk = as_buffer(vectors, np.float32, (n, d))
        cnt = d if self.per_dim else 1
        s = np.empty(cnt, np.float32)
        o = np.empty(cnt, np.float32)
        self.ctx.check(self.ctx.lib.vsk_sq8_train(self.ctx.handle, xp, n, d,
                                                  1 if self.per_dim else 0,
                                                  s.ctypes.data, o.ctypes.data))
        self.scale, self.offset = s, o
        self.dimensions = d
        return s, o

    def _need(self):
        if self.scale is None:
            raise VSKError(-7, "quantizer is not trained")

    def quantizeBatch(self, vectors):
        self._need()
        n, d = int(vectors.shape[0]), int(vectors.shape[1])
        xp, xk = as_buffer(vectors, np.float32, (n, d))
        cp, codes = out_buffer((n, d), np.int8, vectors)
        self.ctx.check(self.ctx.lib.vsk_sq8_encode(
            self.ctx.handle, xp, n, d, 1 if self.per_dim else 0,
            self.scale.ctypes.data, self.offset.ctypes.data, cp))
        return codes

    def dequantize(self, codes):
        """dequantizeFromInt8 (Quantization/ScalarQuantizer.swift:568-580) on the
        GPU (vsk_sq8_decode): (code - offset) / scale."""
        self._need()
        n, d = int(codes.shape[0]), int(codes.shape[1])
        cp, ck = as_buffer(codes, np.int8, (n, d))
        op, out = out_buffer((n, d), np.float32, codes)
        self.ctx.check(self.ctx.lib.vsk_sq8_decode(
            self.ctx.handle, cp, n, d, 1 if self.per_dim else 0,
            self.scale.ctypes.data, self.offset.ctypes.data, op))
        return out


class SQ8Database:
    """Resident int8 code rows (``vsk_sq8``)."""

    def __init__(self, ctx: Context, codes):
        self.ctx = ctx
        self.n, self.d = int(codes.shape[0]), int(codes.shape[1])
        cp, ck = as_buffer(codes, np.int8, (self.n, self.d))
        h = ctypes.c_void_p()
        ctx.check(ctx.lib.vsk_sq8_upload(ctx.handle, cp, self.n, self.d, ctypes.byref(h)))
        self.handle = h

    def search(self, qcodes, k: int):
        """Top-k by int32 score (descending), ties by id: (scores, ids)."""
        nq = int(qcodes.shape[0])
        qp, qk = as_buffer(qcodes, np.int8, (nq, self.d))
        sp, score = out_buffer((nq, k), np.int32, qcodes)
        ip, ids = out_buffer((nq, k), np.int64, qcodes)
        self.ctx.check(self.ctx.lib.vsk_sq8_search(self.ctx.handle, self.handle, qp, nq, k,
                                                   sp, ip))
        return score, ids

    def free(self):
        if getattr(self, "handle", None):
            self.ctx.lib.vsk_sq8_free(self.ctx.handle, self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class ProductQuantizer:
    """PQ with trained codebooks (M, ksub, dsub) and resident codes."""

    @classmethod
    def train(cls, ctx: Context, vectors, M: int, ksub: int = 256, iterations: int = 25,
              seed: int = 0, initMethod: str = "kMeansPlusPlus") -> "ProductQuantizer":
        """ProductQuantizer.train (Quantization/ProductQuantizer.swift:34-64):
        per segment m, trainSegmentCodebook (:270-324) -- k-means with
        maxIterations = iterations (config.trainingIterations), tolerance
        1e-4, k-means++ seeded with the segment index (seed + m here; seed 0
        is the reference's) -- run on the GPU by vsk_kmeans.  The reference
        switches to unseeded mini-batch k-means above 10,000 rows (:287-293);
        full Lloyd iterations are run at every size here."""
        from .clustering import KMeansClustering, KMeansClusteringConfiguration

        x = np.asarray(vectors.cpu().numpy() if _lib._is_torch(vectors) else vectors,
                       np.float32)
        n, d = x.shape
        if d % M:
            raise VSKError(-2, f"dimension {d} is not a multiple of {M} segments")
        if n < ksub:
            raise VSKError(-2, f"insufficient training data: {n} < {ksub}")
        dsub = d // M
        books = np.empty((M, ksub, dsub), np.float32)
        for m in range(M):
            seg = np.ascontiguousarray(x[:, m * dsub:(m + 1) * dsub])
            cfg = KMeansClusteringConfiguration(maxIterations=iterations, tolerance=1e-4,
                                                initMethod=initMethod, seed=seed + m)
            books[m] = KMeansClustering(ctx, cfg).cluster(seg, ksub).centroids
        return cls(ctx, books)

    def __init__(self, ctx: Context, codebooks):
        self.ctx = ctx
        cb = np.ascontiguousarray(codebooks, np.float32)
        if cb.ndim != 3:
            raise VSKError(-4, "codebooks must be (M, ksub, dsub)")
        self.M, self.ksub, self.dsub = cb.shape
        self.d = self.M * self.dsub
        self.codebooks = cb
        h = ctypes.c_void_p()
        ctx.check(ctx.lib.vsk_pq_create(ctx.handle, cb.ctypes.data, self.M, self.ksub,
                                        self.dsub, ctypes.byref(h)))
        self.handle = h

    @classmethod
    def upload(cls, ctx: Context, codebooks, codes) -> "ProductQuantizer":
        """Trained 8-bit codebooks (M, 256, dsub) and resident codes (n, M)
        in one call (``vsk_pq_upload``)."""
        cb = np.ascontiguousarray(codebooks, np.float32)
        if cb.ndim != 3 or cb.shape[1] != 256:
            raise VSKError(-4, "codebooks must be (M, 256, dsub)")
        M, _, dsub = cb.shape
        n = int(codes.shape[0])
        cp, ck = as_buffer(codes, np.uint8, (n, M))
        h = ctypes.c_void_p()
        ctx.check(ctx.lib.vsk_pq_upload(ctx.handle, cb.ctypes.data, cp, n, M, dsub,
                                        ctypes.byref(h)))
        pq = cls.__new__(cls)
        pq.ctx = ctx
        pq.M, pq.ksub, pq.dsub = M, 256, dsub
        pq.d = M * dsub
        pq.codebooks = cb
        pq.handle = h
        return pq

    def encode(self, vectors):
        n = int(vectors.shape[0])
        xp, xk = as_buffer(vectors, np.float32, (n, self.d))
        cp, codes = out_buffer((n, self.M), np.uint8, vectors)
        self.ctx.check(self.ctx.lib.vsk_pq_encode(self.ctx.handle, self.handle, xp, n, cp))
        return codes

    def decode(self, codes):
        """ProductQuantizer.decode (Quantization/ProductQuantizer.swift:142-160)
        on the GPU (vsk_pq_decode): each segment's codeword."""
        n = int(codes.shape[0])
        cp, ck = as_buffer(codes, np.uint8, (n, self.M))
        op, out = out_buffer((n, self.d), np.float32, codes)
        self.ctx.check(self.ctx.lib.vsk_pq_decode(self.ctx.handle, self.handle, cp, n, op))
        return out

    def add(self, codes):
        n = int(codes.shape[0])
        cp, ck = as_buffer(codes, np.uint8, (n, self.M))
        self.ctx.check(self.ctx.lib.vsk_pq_add_codes(self.ctx.handle, self.handle, cp, n))

    def precomputeDistanceTables(self, queries):
        q = queries if len(queries.shape) == 2 else queries.reshape(1, -1)
        nq = int(q.shape[0])
        qp, qk = as_buffer(q, np.float32, (nq, self.d))
        lp, lut = out_buffer((nq, self.M, self.ksub), np.float32, q)
        self.ctx.check(self.ctx.lib.vsk_pq_lut(self.ctx.handle, self.handle, qp, nq, lp))
        return lut

    def search(self, queries, k: int, k_adc: int | None = None, rerank_metric=None,
               rerank_db: VectorDatabase | None = None):
        k_adc = k_adc or k
        nq = int(queries.shape[0])
        qp, qk = as_buffer(queries, np.float32, (nq, self.d))
        dp, dist = out_buffer((nq, k), np.float32, queries)
        ip, ids = out_buffer((nq, k), np.int64, queries)
        m = metric_code(rerank_metric) if rerank_metric is not None else -1
        self.ctx.check(self.ctx.lib.vsk_pq_search(
            self.ctx.handle, self.handle, qp, nq, k_adc, k, m,
            rerank_db.handle if rerank_db is not None else None, dp, ip))
        return dist, ids

    def free(self):
        if getattr(self, "handle", None):
            self.ctx.lib.vsk_pq_free(self.ctx.handle, self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class BinaryQuantizer:
    """quantizeVectors(scheme: .binary) (AccelerateOptimizer.binaryQuantize,
    Acceleration/AccelerateOptimizer.swift:447-481): one bit per dimension,
    x_i > 0, byte i/8 bit i%8 -- encoded on the GPU (vsk_binary_encode)."""

    def __init__(self, ctx: Context):
        self.ctx = ctx

    def quantizeBatch(self, vectors):
        n, d = int(vectors.shape[0]), int(vectors.shape[1])
        xp, xk = as_buffer(vectors, np.float32, (n, d))
        cp, codes = out_buffer((n, (d + 7) // 8), np.uint8, vectors)
        self.ctx.check(self.ctx.lib.vsk_binary_encode(self.ctx.handle, xp, n, d, cp))
        return codes


class BinaryDatabase:
    """Resident binary codes (``vsk_bin``) searched by Hamming distance
    (binaryHammingDistance, QuantizationShaders.metal:285-305)."""

    def __init__(self, ctx: Context, codes, d: int):
        self.ctx = ctx
        self.n, self.d = int(codes.shape[0]), int(d)
        nb = (self.d + 7) // 8
        cp, ck = as_buffer(codes, np.uint8, (self.n, nb))
        h = ctypes.c_void_p()
        ctx.check(ctx.lib.vsk_bin_upload(ctx.handle, cp, self.n, self.d, ctypes.byref(h)))
        self.handle = h

    def search(self, qcodes, k: int):
        """Top-k by Hamming distance, ties by id: (int32 distances, ids)."""
        nq = int(qcodes.shape[0])
        qp, qk = as_buffer(qcodes, np.uint8, (nq, (self.d + 7) // 8))
        dp, dist = out_buffer((nq, k), np.int32, qcodes)
        ip, ids = out_buffer((nq, k), np.int64, qcodes)
        self.ctx.check(self.ctx.lib.vsk_bin_search(self.ctx.handle, self.handle, qp, nq, k,
                                                   dp, ip))
        return dist, ids

    def distances(self, qcodes):
        """Every (query, row) Hamming distance as float32 (nq, n)."""
        nq = int(qcodes.shape[0])
        qp, qk = as_buffer(qcodes, np.uint8, (nq, (self.d + 7) // 8))
        op, out = out_buffer((nq, self.n), np.float32, qcodes)
        self.ctx.check(self.ctx.lib.vsk_bin_distances(self.ctx.handle, self.handle, qp, nq, op))
        return out

    def free(self):
        if getattr(self, "handle", None):
            self.ctx.lib.vsk_bin_free(self.ctx.handle, self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

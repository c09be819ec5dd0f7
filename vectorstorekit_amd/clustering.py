"""``KMeansClustering`` mirror over the C ABI (Clustering/KMeansClustering.swift
of gifton/VectorStoreKit): every Lloyd iteration and the k-means++ seeding run
on the GPU (``vsk_kmeans``).

Reference surface kept: ``KMeansClusteringConfiguration(maxIterations,
tolerance, initMethod, seed)`` (Config/Clustering/
KMeansClusteringConfiguration.swift:8-50, presets ``default``/``fast``/
``accurate``), ``KMeansClustering(configuration).cluster(vectors, k,
weights)`` (:48-113) returning ``ClusteringResult(centroids, assignments,
iterations, converged, inertia)`` (:9-29), and ``ClusteringError`` cases as
``VSKError`` kinds.  ``useMetalAcceleration`` has no meaning here (the GPU
path is the only path).  ``miniBatchCluster`` (:116-174) is not provided:
its batches come from unseeded shuffles that no run can reproduce.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from ._lib import VSKError, as_buffer, out_buffer
from .engine import Context

INIT_RANDOM = 0
INIT_CUSTOM = 1
INIT_PLUSPLUS = 2
_INIT = {"random": INIT_RANDOM, "custom": INIT_CUSTOM, "kMeansPlusPlus": INIT_PLUSPLUS}


class vsk_kmeans_result(ctypes.Structure):
    _fields_ = [("iterations", ctypes.c_int32), ("converged", ctypes.c_int32),
                ("inertia", ctypes.c_float)]


@dataclass
class KMeansClusteringConfiguration:
    """initMethod: "random", "kMeansPlusPlus" or "custom" (then
    ``customCentroids`` holds the k starting centroids).  seed None draws a
    fresh seed per call, as the reference's system generator does."""

    maxIterations: int = 100
    tolerance: float = 1e-4
    initMethod: str = "kMeansPlusPlus"
    seed: int | None = None
    customCentroids: object = field(default=None, repr=False)

    @classmethod
    def default(cls):
        return cls()

    @classmethod
    def fast(cls):
        return cls(maxIterations=50, tolerance=1e-3, initMethod="random")

    @classmethod
    def accurate(cls):
        return cls(maxIterations=200, tolerance=1e-5, initMethod="kMeansPlusPlus")


@dataclass
class ClusteringResult:
    centroids: object      # (k, d) float32 (numpy, or a torch tensor on the inputs' GPU)
    assignments: object    # (n,) int32
    iterations: int
    converged: bool
    inertia: float


class KMeansClustering:
    def __init__(self, ctx: Context, configuration: KMeansClusteringConfiguration | None = None):
        self.ctx = ctx
        self.configuration = configuration or KMeansClusteringConfiguration()
        if self.configuration.initMethod not in _INIT:
            raise VSKError(-2, f"unknown initMethod {self.configuration.initMethod!r}")

    def cluster(self, vectors, k: int, weights=None) -> ClusteringResult:
        cfg = self.configuration
        if vectors.shape[0] == 0:
            raise VSKError(-3, "cannot cluster an empty dataset")
        n, d = int(vectors.shape[0]), int(vectors.shape[1])
        xp, xk = as_buffer(vectors, np.float32, (n, d))
        wp, wk = (as_buffer(weights, np.float32, (n,)) if weights is not None
                  else (None, None))
        method = _INIT[cfg.initMethod]
        cp = ck = None
        if method == INIT_CUSTOM:
            if cfg.customCentroids is None:
                raise VSKError(-2, "custom initialisation needs customCentroids")
            cp, ck = as_buffer(cfg.customCentroids, np.float32)
            if tuple(ck.shape) != (k, d):
                raise VSKError(-2, f"custom centroids count ({ck.shape[0]}) doesn't "
                               f"match k ({k})")
        seed = cfg.seed if cfg.seed is not None else int.from_bytes(os.urandom(8), "little")
        op, cent = out_buffer((k, d), np.float32, vectors)
        ap, assign = out_buffer((n,), np.int32, vectors)
        res = vsk_kmeans_result()
        self.ctx.check(self.ctx.lib.vsk_kmeans(
            self.ctx.handle, xp, n, d, int(k), wp, method, cp, ctypes.c_uint64(seed & (2**64 - 1)),
            int(cfg.maxIterations), float(cfg.tolerance), op, ap, ctypes.byref(res)))
        return ClusteringResult(cent, assign, int(res.iterations), bool(res.converged),
                                float(res.inertia))

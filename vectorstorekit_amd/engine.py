"""Host-side mirror of VectorStoreKit's accelerator surface over the C ABI.

* ``HIPAcceleratorStrategy`` -- the ``ComputeAccelerator`` slot
  (Core/Protocols.swift:11-20; Metal versions in
  API/Strategies/AcceleratorStrategies.swift:20-214): ``identifier``,
  ``requirements``, ``initialize()``, ``capabilities()``.
* ``HIPAccelerationEngine`` -- ``MetalAccelerationEngine``'s distance API
  (Acceleration/MetalAccelerationEngine.swift:76-204):
  ``computeDistances(query, candidates, metric)`` and
  ``batchComputeDistances(queries, candidates, metric, topK)``, plus
  ``search`` which also returns the ids (the reference returns distances
  only).
* ``VectorDatabase`` -- rows resident in HBM (``vsk_db``).

Paths in citations are relative to Sources/VectorStoreKit/ of
gifton/VectorStoreKit.  Every call goes through libvsk_hip.so; there is no
CPU fallback.
"""
from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import VSKError, as_buffer, check, load_library, out_buffer


class DistanceMetric(str, enum.Enum):
    """``DistanceMetric`` raw values (Core/SearchTypes.swift:105-112) for the
    five metrics UnifiedDistanceComputation evaluates (the four hot-path
    ones and hamming), plus the squared-L2 and pre-normalised cosine forms
    of the reference's kernels."""

    euclidean = "euclidean"
    cosine = "cosine"
    dotProduct = "dotProduct"
    manhattan = "manhattan"
    hamming = "hamming"
    euclideanSquared = "euclideanSquared"
    cosineNormalized = "cosineNormalized"

    @property
    def code(self) -> int:
        return _METRIC_CODES[self]


_METRIC_CODES = {
    DistanceMetric.euclideanSquared: _lib.METRIC_L2SQ,
    DistanceMetric.euclidean: _lib.METRIC_L2,
    DistanceMetric.cosine: _lib.METRIC_COSINE,
    DistanceMetric.cosineNormalized: _lib.METRIC_COSINE_NORMALIZED,
    DistanceMetric.dotProduct: _lib.METRIC_DOT,
    DistanceMetric.manhattan: _lib.METRIC_L1,
    DistanceMetric.hamming: _lib.METRIC_HAMMING,
}


def _to_host(a):
    return a.cpu().numpy() if _lib._is_torch(a) else a


def metric_code(metric) -> int:
    if isinstance(metric, int):
        return metric
    return DistanceMetric(metric).code


class DistanceComputeBackend(str, enum.Enum):
    """``DistanceComputeBackend`` (Config/Core/StoreConfiguration.swift:145-166)
    with the ``hip`` case this build adds.  ``selectOptimal`` keeps the
    reference's heuristics for its own backends and takes ``hip`` whenever a
    HIP device serves the store: this build has no CPU product path, so small
    batches run on the GPU too (the reference sends them to Accelerate)."""

    metal = "metal"
    accelerate = "accelerate"
    simd = "simd"
    auto = "auto"
    hip = "hip"

    def selectOptimal(self, dimension: int, candidateCount: int,
                      hipAvailable: bool = True) -> "DistanceComputeBackend":
        if self != DistanceComputeBackend.auto:
            return self
        if hipAvailable:
            return DistanceComputeBackend.hip
        if candidateCount > 1000:
            return DistanceComputeBackend.metal
        return (DistanceComputeBackend.simd if dimension == 512
                else DistanceComputeBackend.accelerate)


@dataclass(frozen=True)
class HIPAccelerationConfiguration:
    """``MetalComputeConfiguration`` (Config/Acceleration/
    MetalComputeConfiguration.swift:8-46) for the HIP device, applied to a
    context by ``vsk_configure``.

    * ``kernel``: "auto" (the bf16 screen where it is exact and pays),
      "exact" (exact scans only), "screen" (the screen at every size),
      "bf16x3" / "fp32" (tolerance-path flat kernels);
    * ``enableProfiling``: per-kernel HIP-event timing;
    * ``maxTileBytes``: the working-buffer limit a query batch stays under
      (0: the default, 2 GiB of candidate keys); searches chunk their
      queries under it, as MetalDistanceCompute chunks under its buffer
      limit (Acceleration/Metal/MetalDistanceCompute.swift:371-380);
    * ``minBatchSizeForGPU``: kept for the reference's API; nothing is routed
      to a CPU path by it here."""

    kernel: str = "auto"
    enableProfiling: bool = False
    maxTileBytes: int = 0
    minBatchSizeForGPU: int = 1000

    _KERNELS = {"auto": 0, "exact": 1, "screen": 2, "bf16x3": 3, "fp32": 4}

    def validate(self):
        if self.kernel not in self._KERNELS:
            raise VSKError(-2, f"unknown kernel choice {self.kernel!r}")
        if self.maxTileBytes < 0 or self.minBatchSizeForGPU <= 0:
            raise VSKError(-2, "maxTileBytes must be >= 0 and minBatchSizeForGPU positive")

    @classmethod
    def research(cls):
        return cls(enableProfiling=True, minBatchSizeForGPU=500)

    @classmethod
    def efficient(cls):
        return cls(enableProfiling=False, minBatchSizeForGPU=2000)


class Context:
    """One ``vsk_ctx``: a device and the HIP stream every call runs on."""

    def __init__(self, device: int = 0, configuration: HIPAccelerationConfiguration | None = None):
        self.lib = load_library()
        h = ctypes.c_void_p()
        st = self.lib.vsk_create(device, ctypes.byref(h))
        if st != 0:
            raise VSKError(st, f"cannot open HIP device {device}")
        self.handle = h
        self.device = device
        if configuration is not None:
            self.configure(configuration)

    def configure(self, configuration: HIPAccelerationConfiguration):
        """Apply a configuration to later calls (``vsk_configure``)."""
        configuration.validate()
        cfg = _lib.vsk_config(configuration._KERNELS[configuration.kernel],
                              1 if configuration.enableProfiling else 0,
                              int(configuration.maxTileBytes))
        self.check(self.lib.vsk_configure(self.handle, ctypes.byref(cfg)))

    def configuration(self) -> HIPAccelerationConfiguration:
        cfg = _lib.vsk_config()
        self.check(self.lib.vsk_get_config(self.handle, ctypes.byref(cfg)))
        names = {v: k for k, v in HIPAccelerationConfiguration._KERNELS.items()}
        return HIPAccelerationConfiguration(kernel=names[cfg.kernel],
                                            enableProfiling=bool(cfg.enable_profiling),
                                            maxTileBytes=int(cfg.max_tile_bytes))

    def close(self):
        if getattr(self, "handle", None):
            self.lib.vsk_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def check(self, status):
        check(self.handle, status)

    @property
    def stream(self) -> int:
        return self.lib.vsk_stream(self.handle) or 0

    @property
    def last_kernel_ms(self) -> float:
        return float(self.lib.vsk_last_kernel_ms(self.handle))

    def last_sync_count(self) -> int:
        """Host waits for the stream in the last call (``vsk_last_sync_count``)."""
        return int(self.lib.vsk_last_sync_count(self.handle))

    def measure_peaks(self) -> dict:
        """Measured ceilings of the device (``vsk_measure_peaks``): dense
        bf16 TFLOP/s, dense int8 TOP/s, HBM copy GB/s (read plus written)
        and HBM read GB/s."""
        from ._lib import vsk_peaks

        pk = vsk_peaks()
        self.check(self.lib.vsk_measure_peaks(self.handle, ctypes.byref(pk)))
        return {"bf16_tflops": pk.bf16_tflops, "int8_tops": pk.int8_tops,
                "hbm_gbs": pk.hbm_gbs, "hbm_read_gbs": pk.hbm_read_gbs}

    def last_screen_redo(self, tier: int) -> np.ndarray:
        """Query indices the last flat search redid in the screen's tier 1
        (wider screen) or tier 2 (exact scan over every row)."""
        cnt = ctypes.c_int64()
        self.check(self.lib.vsk_last_screen_redo(self.handle, tier, None, 0, ctypes.byref(cnt)))
        out = np.empty(cnt.value, np.int64)
        if cnt.value:
            self.check(self.lib.vsk_last_screen_redo(self.handle, tier, out.ctypes.data,
                                                     cnt.value, ctypes.byref(cnt)))
        return out

    def capabilities(self) -> dict:
        caps = _lib.vsk_caps()
        self.check(self.lib.vsk_device_info(self.handle, ctypes.byref(caps)))
        return {
            "name": caps.name.decode(),
            "arch": caps.arch.decode(),
            "device": caps.device,
            "compute_units": caps.compute_units,
            "wavefront_size": caps.wavefront_size,
            "lds_bytes_per_block": caps.lds_bytes_per_block,
            "global_mem_bytes": caps.global_mem_bytes,
            "clock_khz": caps.clock_khz,
            "memory_clock_khz": caps.memory_clock_khz,
            "memory_bus_width_bits": caps.memory_bus_width_bits,
        }

    # per-kernel HIP-event timing
    def profile(self, on: bool = True):
        self.check(self.lib.vsk_profile_enable(self.handle, 1 if on else 0))

    def profile_only(self, names=None):
        """Time only the timers named in ``names`` (an iterable of names;
        None or empty: all of them again).  Device-side work counts are not
        read back meanwhile (their stats report 0 work)."""
        arg = ",".join(names).encode() if names else None
        self.check(self.lib.vsk_profile_only(self.handle, arg))

    def profile_reset(self):
        self.check(self.lib.vsk_profile_reset(self.handle))

    def profile_stats(self) -> dict:
        out = {}
        for i in range(self.lib.vsk_profile_count(self.handle)):
            s = _lib.vsk_kernel_stat()
            self.check(self.lib.vsk_profile_get(self.handle, i, ctypes.byref(s)))
            out[s.name.decode()] = (int(s.launches), float(s.total_ms), float(s.work))
        return out


class VectorDatabase:
    """Database rows resident in HBM (``vsk_db_upload_f32``).  ``vectors``
    is an (n, d) float32 numpy array or torch tensor (host or device)."""

    def __init__(self, ctx: Context, vectors, normalize: bool = False):
        self.ctx = ctx
        shape = tuple(vectors.shape)
        if len(shape) != 2:
            raise VSKError(-4, "vectors must be 2-D (n, d)")
        self.n, self.d = int(shape[0]), int(shape[1])
        ptr, keep = as_buffer(vectors, np.float32)
        h = ctypes.c_void_p()
        ctx.check(ctx.lib.vsk_db_upload_f32(ctx.handle, ptr, self.n, self.d,
                                            _lib.DB_NORMALIZE if normalize else 0,
                                            ctypes.byref(h)))
        del keep
        self.handle = h

    def free(self):
        if getattr(self, "handle", None):
            self.ctx.lib.vsk_db_free(self.ctx.handle, self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def read(self, row0: int = 0, count: int | None = None) -> np.ndarray:
        count = self.n - row0 if count is None else count
        out = np.empty((count, self.d), np.float32)
        self.ctx.check(self.ctx.lib.vsk_db_read_f32(self.ctx.handle, self.handle, row0,
                                                    count, out.ctypes.data))
        return out

    def search(self, queries, k: int, metric="euclidean", allow=None):
        """Exact top-k: (distances [nq, k] float32, ids [nq, k] int64),
        ascending (distance, id).  Outputs are torch tensors on the device
        when ``queries`` is a CUDA tensor, else numpy arrays.  ``allow``
        (optional) keeps only some rows as candidates: a boolean array over
        the rows or the allowed row indices (``vsk_search_flat_filtered``)."""
        nq = int(queries.shape[0])
        qp, qk = as_buffer(queries, np.float32, (nq, self.d))
        dp, dist = out_buffer((nq, k), np.float32, queries)
        ip, ids = out_buffer((nq, k), np.int64, queries)
        if allow is None:
            self.ctx.check(self.ctx.lib.vsk_search_flat(self.ctx.handle, self.handle, qp, nq,
                                                        k, metric_code(metric), dp, ip))
        else:
            a = np.asarray(allow)
            bm = _lib.row_bitmap(a, self.n)
            nbits = int(a.size) if a.dtype == np.bool_ else self.n
            self.ctx.check(self.ctx.lib.vsk_search_flat_filtered(
                self.ctx.handle, self.handle, qp, nq, k, metric_code(metric), bm.ctypes.data,
                nbits, dp, ip))
        del qk
        return dist, ids

    def distances(self, queries, metric="euclidean"):
        """Full distance matrix [nq, n]."""
        nq = int(queries.shape[0])
        qp, qk = as_buffer(queries, np.float32, (nq, self.d))
        mp, mat = out_buffer((nq, self.n), np.float32, queries)
        self.ctx.check(self.ctx.lib.vsk_distances(self.ctx.handle, self.handle, qp, nq,
                                                  metric_code(metric), mp))
        del qk
        return mat


@dataclass(frozen=True)
class HardwareRequirements:
    """``HardwareRequirements`` of the accelerator slot."""

    minimumMemory: int = 0
    requiredComputeUnits: int = 1
    requiredFeatures: tuple = ("gfx950",)


class HIPAcceleratorStrategy:
    """``ComputeAccelerator`` conformance for HIP (Core/Protocols.swift:11-20):
    ``initialize()`` returns the device context, ``capabilities()`` its
    description.  This is what ``accelerate(using:)`` receives."""

    identifier = "hip-gfx950"
    requirements = HardwareRequirements()

    def __init__(self, device: int = 0,
                 configuration: HIPAccelerationConfiguration | None = None):
        self.device = device
        self.configuration = configuration
        self._ctx: Context | None = None

    def initialize(self) -> Context:
        if self._ctx is None:
            self._ctx = Context(self.device, self.configuration)
        return self._ctx

    def capabilities(self) -> dict:
        return self.initialize().capabilities()


@dataclass(frozen=True)
class QuantizationScheme:
    """``QuantizationScheme`` (Core/VectorTypes.swift:474-505): ``kind`` is its
    raw value ("scalar", "product", "binary", "vector", "learned", "none")."""

    kind: str
    bits: int = 8
    segments: int = 0

    @staticmethod
    def scalar(bits: int = 8) -> "QuantizationScheme":
        return QuantizationScheme("scalar", bits)

    @staticmethod
    def product(segments: int, bits: int = 8) -> "QuantizationScheme":
        return QuantizationScheme("product", bits, segments)

    @staticmethod
    def binary() -> "QuantizationScheme":
        return QuantizationScheme("binary", 1)

    @staticmethod
    def none() -> "QuantizationScheme":
        return QuantizationScheme("none", 32)


@dataclass(frozen=True)
class QuantizationParameters:
    """``QuantizationParameters`` (Core/VectorTypes.swift:508-540)."""

    trainingIterations: int = 25
    useAsymmetricDistance: bool = True
    useOptimizedLayout: bool = True
    compressionTarget: float | None = None
    precision: int = 8
    centroids: int | None = None
    subvectors: int | None = None
    seed: int = 0


@dataclass(frozen=True)
class QuantizationMetadata:
    scheme: QuantizationScheme
    originalDimensions: int
    compressionRatio: float


@dataclass(frozen=True)
class QuantizedVector:
    """``QuantizedVector`` (Core/VectorTypes.swift:543-580): the codes of one
    vector and its metadata; ``scale`` / ``minimum`` carry the per-vector
    parameters of the scalar scheme (the reference computes them and drops
    them, AccelerateOptimizer.swift:415-419)."""

    codes: bytes
    metadata: QuantizationMetadata
    scale: float | None = None
    minimum: float | None = None

    @property
    def originalDimensions(self) -> int:
        return self.metadata.originalDimensions

    @property
    def scheme(self) -> QuantizationScheme:
        return self.metadata.scheme


class HIPAccelerationEngine:
    """``MetalAccelerationEngine``'s distance and quantization API on the HIP
    library (Acceleration/MetalAccelerationEngine.swift:76-262).  Candidates
    may be a ``VectorDatabase`` (resident) or an array uploaded for the call
    and freed when it returns."""

    def __init__(self, device: int | Context = 0):
        self.ctx = device if isinstance(device, Context) else Context(device)

    def _db(self, candidates):
        """(database, uploaded_here): the candidates as a resident database."""
        if isinstance(candidates, VectorDatabase):
            return candidates, False
        if len(candidates) == 0:
            raise VSKError(-3, "candidates is empty")
        return VectorDatabase(self.ctx, np.asarray(candidates, np.float32)
                              if not _lib._is_torch(candidates) else candidates), True

    def _with_db(self, candidates, fn):
        db, temp = self._db(candidates)
        try:
            return fn(db)
        finally:
            if temp:
                db.free()

    def computeDistances(self, query, candidates, metric="euclidean"):
        """Distances from one query to every candidate (:76-136)."""
        q = np.asarray(query, np.float32).reshape(1, -1) if not _lib._is_torch(query) \
            else query.reshape(1, -1)
        return self._with_db(candidates, lambda db: db.distances(q, metric)[0])

    def batchComputeDistances(self, queries, candidates, metric="euclidean", topK=None):
        """Per query: all distances (topK None) or the topK smallest,
        ascending (:139-204)."""
        def run(db):
            if topK is None:
                return db.distances(queries, metric)
            dist, _ = db.search(queries, min(int(topK), db.n), metric)
            return dist

        return self._with_db(candidates, run)

    def search(self, queries, candidates, k: int, metric="euclidean"):
        """Top-k distances and ids."""
        return self._with_db(candidates, lambda db: db.search(queries, k, metric))

    def quantizeVectors(self, vectors, scheme: QuantizationScheme,
                        parameters: QuantizationParameters | None = None):
        """``quantizeVectors(vectors:scheme:parameters:)`` (:234-262), on the
        device, with the reference CPU path's semantics
        (AccelerateOptimizer.quantizeVectors, Acceleration/
        AccelerateOptimizer.swift:217-247):

        * scalar(bits): per-vector min/max, uint8 codes truncated
          (``vsk_scalar_quantize_u8``, :387-430);
        * binary: one bit per dimension, x > 0 (``vsk_binary_encode``,
          :447-481);
        * product(segments, bits): codebooks trained by k-means
          (``parameters.trainingIterations``, 2^bits codewords) and the
          vectors encoded, one byte per segment (``ProductQuantizer``).  The
          reference's CPU path is a placeholder that falls back to scalar
          quantization (:432-445); this is the product quantizer it names;
        * any other scheme: the raw fp32 bytes (the reference's default
          branch, :233-245).

        Returns a list of ``QuantizedVector``."""
        parameters = parameters or QuantizationParameters()
        x = vectors
        if not _lib._is_torch(x):
            x = np.ascontiguousarray(np.asarray(x, np.float32))
        n, d = int(x.shape[0]), int(x.shape[1])
        if n == 0:
            raise VSKError(-3, "no vectors")
        if scheme.kind == "scalar":
            xp, xk = as_buffer(x, np.float32, (n, d))
            codes = np.empty((n, d), np.uint8)
            sc = np.empty(n, np.float32)
            mn = np.empty(n, np.float32)
            self.ctx.check(self.ctx.lib.vsk_scalar_quantize_u8(
                self.ctx.handle, xp, n, d, scheme.bits, codes.ctypes.data, sc.ctypes.data,
                mn.ctypes.data))
            ratio = d * 4.0 / (d + 8)
            meta = QuantizationMetadata(scheme, d, ratio)
            return [QuantizedVector(codes[i].tobytes(), meta, float(sc[i]), float(mn[i]))
                    for i in range(n)]
        if scheme.kind == "binary":
            from .quantization import BinaryQuantizer

            codes = np.asarray(_to_host(BinaryQuantizer(self.ctx).quantizeBatch(x)))
            meta = QuantizationMetadata(scheme, d, d * 4.0 / codes.shape[1])
            return [QuantizedVector(codes[i].tobytes(), meta) for i in range(n)]
        if scheme.kind == "product":
            from .quantization import ProductQuantizer

            M = scheme.segments or parameters.subvectors
            if not M or d % M:
                raise VSKError(-2, "product quantization needs segments dividing the dimension")
            ksub = min(parameters.centroids or (1 << scheme.bits), 256)
            pq = ProductQuantizer.train(self.ctx, x, M, ksub,
                                        iterations=parameters.trainingIterations,
                                        seed=parameters.seed)
            try:
                codes = np.asarray(_to_host(pq.encode(x)))
            finally:
                pq.free()
            meta = QuantizationMetadata(scheme, d, d * 4.0 / M)
            return [QuantizedVector(codes[i].tobytes(), meta) for i in range(n)]
        raw = np.asarray(_to_host(x), np.float32)
        meta = QuantizationMetadata(scheme, d, 1.0)
        return [QuantizedVector(raw[i].tobytes(), meta) for i in range(n)]

    def computeDistanceMatrix(self, vectorsA, vectorsB=None, metric="euclidean"):
        """MetalDistanceMatrix.computeDistanceMatrix (Acceleration/Metal/
        MetalDistanceMatrix.swift:49-120): the |A| x |B| distance matrix;
        vectorsB None is the symmetric matrix of A, whose upper triangle
        (i <= j) is mirrored below the diagonal as the reference does
        (:340-385).  Every metric is summed in the reference's order on the
        exact kernel, so (i, j) and (j, i) are equal already."""
        b = vectorsA if vectorsB is None else vectorsB
        m = self._with_db(b, lambda db: db.distances(vectorsA, metric))
        if vectorsB is None:
            if _lib._is_torch(m):
                import torch

                m = torch.triu(m) + torch.triu(m, 1).T
            else:
                m = np.triu(m) + np.triu(m, 1).T
        return m

    def matrixMultiply(self, matrixA, matrixB):
        """MetalAccelerationEngine.matrixMultiply(matrixA:matrixB:)
        (Acceleration/MetalAccelerationEngine.swift:209-229): A (m x k) times
        B (k x n) as an m x n fp32 matrix (``vsk_matrix_multiply``).  Each
        entry is summed over k in order from 0, a product and then a sum, as
        the reference's CPU loop adds it (Acceleration/Metal/
        MetalMatrixCompute.swift:791-806).  A column count of A that differs
        from B's row count raises (the reference's
        MetalMatrixError.dimensionMismatch, MetalAccelerationEngine.swift:
        491-496)."""
        a = matrixA if _lib._is_torch(matrixA) else np.asarray(matrixA, np.float32)
        b = matrixB if _lib._is_torch(matrixB) else np.asarray(matrixB, np.float32)
        if a.ndim != 2 or b.ndim != 2:
            raise VSKError(-2, "matrixMultiply takes two 2-d matrices")
        m, k = int(a.shape[0]), int(a.shape[1])
        if int(b.shape[0]) != k:
            raise VSKError(-4, f"dimension mismatch: a is {m} x {k}, b is "
                               f"{int(b.shape[0])} x {int(b.shape[1])}")
        n = int(b.shape[1])
        ap, ak = as_buffer(a, np.float32, (m, k))
        bp, bk = as_buffer(b, np.float32, (k, n))
        cp, c = out_buffer((m, n), np.float32, a)
        self.ctx.check(self.ctx.lib.vsk_matrix_multiply(self.ctx.handle, ap, m, k, bp, n, cp))
        del ak, bk
        return c

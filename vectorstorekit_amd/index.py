"""``VectorIndex`` conformance of the GPU IVF index: the Python twin of the
Swift ``HIPIVFIndex`` a maintainer adds to VectorStoreKit, making the same C
calls in the same order.

Reference surface (paths relative to Sources/VectorStoreKit/ of
gifton/VectorStoreKit):

* ``VectorIndex.insert(_:) -> InsertResult`` and
  ``search(query:k:strategy:filter:) -> [SearchResult<Metadata>]``
  (Core/Protocols.swift:107-121), as ``IVFIndex`` implements them
  (Indexes/IVFIndex.swift:80-202): insert appends to the nearest centroid's
  list (``vsk_ivf_add``); search probes ``numberOfProbes`` lists, or every
  list for ``.exact`` (:551-554), filters the probed candidates (:161-165),
  ranks the rest by sqrt-L2 with the stable sort's tie order and returns the
  first k (``vsk_ivf_search`` / ``vsk_ivf_search_filtered``).
* ``SearchResult`` (Core/SearchTypes.swift:11-55), as
  ``createSimpleSearchResult`` fills it (Indexes/SearchResultHelpers.swift:
  8-60): id, distance, metadata, tier, confidence, the index algorithm.
* ``InsertResult`` (Core/Protocols.swift:411-423), ``VectorEntry``
  (Core/VectorTypes.swift:23-60), ``SearchStrategy`` (Core/SearchTypes.swift:
  326-437).
* ``delete``/``contains``/``update`` (Indexes/IVFIndex.swift:204-234):
  delete removes one stored row of the id from its list (``vsk_ivf_remove``).
* ``export``/``import`` (Core/Protocols.swift): the whole index as one
  ``vsk_ivf_save`` file, the rows' VectorIDs and metadata in its metadata.

Row ids on the device are the insertion order (0, 1, 2, ...; a removed
row's id is not reused); the index keeps the ``VectorID`` strings and the
metadata of each row on the host, as ``IVFIndex`` keeps them in its
``StoredVector``s.
"""
from __future__ import annotations

import enum
import os
import tempfile
import time
from dataclasses import dataclass
from typing import Any, Callable

import numpy as np

from ._lib import MAX_K, VSKError
from .engine import HIPAcceleratorStrategy
from .ivf import IVFConfiguration, IVFIndex


class SearchStrategy(str, enum.Enum):
    """``SearchStrategy`` cases IVFIndex distinguishes (.exact probes every
    list; the others probe numberOfProbes, Indexes/IVFIndex.swift:551-558)."""

    exact = "exact"
    approximate = "approximate"
    adaptive = "adaptive"
    learned = "learned"
    hybrid = "hybrid"
    anytime = "anytime"
    multimodal = "multimodal"


@dataclass(frozen=True)
class VectorEntry:
    id: str
    vector: Any
    metadata: Any = None


@dataclass(frozen=True)
class InsertResult:
    success: bool
    insertTime: float
    memoryImpact: int
    indexReorganization: bool


@dataclass(frozen=True)
class SearchResult:
    """``SearchResult<Metadata>`` with the fields createSimpleSearchResult
    sets (distance = sqrt-L2, tier .hot, confidence 1, algorithm "IVF")."""

    id: str
    distance: float
    metadata: Any
    tier: str = "hot"
    confidence: float = 1.0
    indexAlgorithm: str = "IVF"


class HIPIVFIndex:
    """IVF-Flat ``VectorIndex`` on one GPU (``IVFIndex`` semantics).

    ``filter`` in ``search`` is a predicate ``filter(id, metadata) -> bool``
    standing in for ``SearchFilter`` + ``FilterEvaluator``.  As in the
    reference it is evaluated on the probed lists' rows only, and the rows it
    rejects are left out before the ranking (a bitmap the device applies in
    its scans), so the k results are exact at any selectivity.

    An id inserted twice is stored twice (the reference appends both copies):
    ``delete`` removes one copy per call -- the one first in list order
    (lists by index, rows in list order; the reference's iteration order over
    its lists is a Dictionary's, which is unspecified) -- and ``contains``
    holds while a copy remains.

    ``trainingSamples`` or ``centroids`` (optional) train the index at
    creation, so an index made by an ``IndexingStrategy`` can take inserts
    through ``VectorStore``'s public API."""

    def __init__(self, accelerator: HIPAcceleratorStrategy, configuration: IVFConfiguration,
                 trainingSamples=None, centroids=None):
        self.accelerator = accelerator
        self.configuration = configuration
        self.ivf = IVFIndex(accelerator.initialize(), configuration)
        self._reset()
        if centroids is not None:
            self.ivf.set_centroids(np.asarray(centroids, np.float32))
        elif trainingSamples is not None:
            self.train(trainingSamples)

    def _reset(self):
        self._stored: list = []  # device id -> (VectorID, metadata), None once removed
        self._rows_of: dict[str, list[int]] = {}  # VectorID -> its stored device ids
        self._count = 0
        self._lists = None  # (ids in list order, offsets), until the lists change

    # ---- VectorIndex properties
    @property
    def count(self) -> int:
        return self._count

    @property
    def capacity(self) -> int:
        return 2 ** 31 - 1

    @property
    def isOptimized(self) -> bool:
        return self.ivf.trained

    # ---- IVF-specific
    def train(self, on):
        """IVFIndex.train(on:) (:397-446): k-means on the device; the lists
        start empty."""
        res = self.ivf.train(np.asarray(on, np.float32))
        self._reset()
        return res

    def _list_ids(self):
        if self._lists is None:
            self._lists = self.ivf.listIds()
        return self._lists

    # ---- core operations
    def insert(self, entry: VectorEntry) -> InsertResult:
        t0 = time.perf_counter()
        if not self.ivf.trained:
            raise VSKError(-7, "IVF index is not trained")
        v = np.ascontiguousarray(np.asarray(entry.vector, np.float32).reshape(1, -1))
        self.ivf.insert(v)  # vsk_ivf_add, ids = the running row count
        self._add_host(entry.id, entry.metadata)
        return InsertResult(True, time.perf_counter() - t0, v.nbytes, False)

    def insertBatch(self, entries) -> list[InsertResult]:
        """``insert`` of every entry, in order, with one ``vsk_ivf_add``."""
        t0 = time.perf_counter()
        if not self.ivf.trained:
            raise VSKError(-7, "IVF index is not trained")
        entries = list(entries)
        if not entries:
            return []
        x = np.ascontiguousarray(np.stack([np.asarray(e.vector, np.float32).reshape(-1)
                                           for e in entries]))
        self.ivf.insert(x)
        for e in entries:
            self._add_host(e.id, e.metadata)
        dt = (time.perf_counter() - t0) / len(entries)
        return [InsertResult(True, dt, x.shape[1] * 4, False) for _ in entries]

    def _add_host(self, vid, metadata):
        self._rows_of.setdefault(vid, []).append(len(self._stored))
        self._stored.append((vid, metadata))
        self._count += 1
        self._lists = None

    def search(self, query, k: int, strategy: SearchStrategy = SearchStrategy.adaptive,
               filter: Callable[[str, Any], bool] | None = None) -> list[SearchResult]:
        if not self.ivf.trained:
            raise VSKError(-7, "IVF index is not trained")
        strategy = SearchStrategy(strategy)
        nprobe = (self.configuration.numberOfCentroids if strategy == SearchStrategy.exact
                  else self.configuration.numberOfProbes)
        if k <= 0:
            return []
        if k > MAX_K:
            raise VSKError(-9, f"k = {k} exceeds VSK_MAX_K = {MAX_K}")
        q = np.ascontiguousarray(np.asarray(query, np.float32).reshape(1, -1))
        if filter is None:
            dist, ids = self.ivf.search(q, k, nprobe=nprobe)  # vsk_ivf_search
        else:
            allow = self._filter_bits(q, nprobe, filter)
            dist, ids = self.ivf.search(q, k, nprobe=nprobe, allow=allow)
        out = []
        for dv, row in zip(np.asarray(dist)[0].tolist(), np.asarray(ids)[0].tolist()):
            if row < 0:
                break
            vid, meta = self._stored[row]
            out.append(SearchResult(vid, float(dv), meta))
        return out

    def _filter_bits(self, q, nprobe, filter) -> np.ndarray:
        """The filter over the query's probed candidates (applyFilter,
        :161-165): a boolean array over the device ids."""
        ids, off = self._list_ids()
        if nprobe >= self.configuration.numberOfCentroids:
            cand = ids
        else:
            probes = np.asarray(self.ivf.probe(q, nprobe))[0]
            cand = np.concatenate([ids[off[l]:off[l + 1]] for l in probes if l >= 0] or
                                  [np.empty(0, np.int64)])
        ok = np.zeros(len(self._stored), np.bool_)
        for row in cand.tolist():
            vid, meta = self._stored[row]
            if filter(vid, meta):
                ok[row] = True
        return ok

    def update(self, id: str, vector=None, metadata=None) -> bool:
        return False  # IVFIndex.update (:204-208)

    def delete(self, id: str) -> bool:
        rows = self._rows_of.get(id)
        if not rows:
            return False
        row = rows[0]
        if len(rows) > 1:
            lids, _ = self._list_ids()
            pos = {int(r): i for i, r in enumerate(lids.tolist()) if r in set(rows)}
            row = min(rows, key=lambda r: pos[r])
        if self.ivf.remove([row]) != 1:
            raise VSKError(-6, f"row {row} of {id!r} was not in the index")
        rows.remove(row)
        if not rows:
            del self._rows_of[id]
        self._stored[row] = None
        self._count -= 1
        self._lists = None
        return True

    def contains(self, id: str) -> bool:
        return bool(self._rows_of.get(id))

    # ---- persistence: the whole index in one file
    def export(self) -> bytes:
        """The index as one ``vsk_ivf_save`` file; the rows' VectorIDs and
        metadata (JSON-serialisable, as the reference's Codable metadata)
        travel in the file's metadata."""
        rows = [[i, s[0], s[1]] for i, s in enumerate(self._stored) if s is not None]
        fd, path = tempfile.mkstemp(suffix=".vskivf")
        os.close(fd)
        try:
            self.ivf.save(path, extra={"rows": rows, "next": len(self._stored)})
            with open(path, "rb") as f:
                return f.read()
        finally:
            os.unlink(path)

    def import_(self, data: bytes):
        """``import(data:format:)``: the index an ``export`` wrote, with its
        VectorIDs and metadata."""
        fd, path = tempfile.mkstemp(suffix=".vskivf")
        try:
            with os.fdopen(fd, "wb") as f:
                f.write(data)
            loaded = IVFIndex.load(self.ivf.ctx, path)
        finally:
            os.unlink(path)
        extra = loaded.savedExtra or {}
        self.ivf.free()
        self.ivf = loaded
        self.configuration = loaded.configuration
        self._reset()
        self._stored = [None] * int(extra.get("next", 0))
        for i, vid, meta in extra.get("rows", []):
            self._stored[i] = (vid, meta)
            self._rows_of.setdefault(vid, []).append(i)
            self._count += 1


class HIPIVFIndexingStrategy:
    """``IndexingStrategy`` whose ``createIndex()`` returns a ``HIPIVFIndex``
    (the HIP twin of IVFIndexingStrategy, API/Strategies/
    IndexingStrategies.swift:230-272).  ``trainingSamples`` or
    ``centroids`` make the created index trained, so inserts and searches
    work through the store's public API (the reference's IVFIndexingStrategy
    returns an untrained index, whose insert throws notTrained)."""

    identifier = "ivf-hip"

    def __init__(self, accelerator: HIPAcceleratorStrategy, dimensions: int,
                 numClusters: int = 1024, nprobe: int = 16,
                 configuration: IVFConfiguration | None = None, trainingSamples=None,
                 centroids=None):
        self.accelerator = accelerator
        self.configuration = configuration or IVFConfiguration(
            dimensions=dimensions, numberOfCentroids=numClusters, numberOfProbes=nprobe)
        self.trainingSamples = trainingSamples
        self.centroids = centroids

    def createIndex(self) -> HIPIVFIndex:
        return HIPIVFIndex(self.accelerator, self.configuration,
                           trainingSamples=self.trainingSamples, centroids=self.centroids)

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
  list for ``.exact`` (:551-554), ranks the union by sqrt-L2 with the stable
  sort's tie order and returns the first k (``vsk_ivf_search``).
* ``SearchResult`` (Core/SearchTypes.swift:11-55), as
  ``createSimpleSearchResult`` fills it (Indexes/SearchResultHelpers.swift:
  8-60): id, distance, metadata, tier, confidence, the index algorithm.
* ``InsertResult`` (Core/Protocols.swift:411-423), ``VectorEntry``
  (Core/VectorTypes.swift:23-60), ``SearchStrategy`` (Core/SearchTypes.swift:
  326-437).
* ``delete``/``contains``/``update`` (Indexes/IVFIndex.swift:204-234):
  deletion marks the id; a search skips marked rows (see ``search``).

Row ids on the device are the insertion order; the index keeps the
``VectorID`` strings and the metadata of each row on the host, as
``IVFIndex`` keeps them in its ``StoredVector``s.
"""
from __future__ import annotations

import enum
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
    standing in for ``SearchFilter`` + ``FilterEvaluator``.  The reference
    filters the probed candidates and then sorts; here the device returns
    the probed candidates in sorted order and the host drops rows that are
    deleted or fail the filter, asking for 2x more until k survive or every
    candidate was returned -- the same k results.  Past ``VSK_MAX_K``
    candidates per query the survivors found so far are returned."""

    def __init__(self, accelerator: HIPAcceleratorStrategy, configuration: IVFConfiguration):
        self.accelerator = accelerator
        self.configuration = configuration
        self.ivf = IVFIndex(accelerator.initialize(), configuration)
        self._ids: list[str] = []
        self._meta: list[Any] = []
        self._row_of: dict[str, int] = {}
        self._deleted: set[int] = set()

    # ---- VectorIndex properties
    @property
    def count(self) -> int:
        return len(self._ids) - len(self._deleted)

    @property
    def capacity(self) -> int:
        return 2 ** 31 - 1

    @property
    def isOptimized(self) -> bool:
        return self.ivf.trained

    # ---- IVF-specific
    def train(self, on):
        """IVFIndex.train(on:) (:397-446): k-means on the device."""
        return self.ivf.train(np.asarray(on, np.float32))

    # ---- core operations
    def insert(self, entry: VectorEntry) -> InsertResult:
        t0 = time.perf_counter()
        if not self.ivf.trained:
            raise VSKError(-7, "IVF index is not trained")
        v = np.ascontiguousarray(np.asarray(entry.vector, np.float32).reshape(1, -1))
        self.ivf.insert(v)  # vsk_ivf_add, ids = the running row count
        self._row_of[entry.id] = len(self._ids)
        self._ids.append(entry.id)
        self._meta.append(entry.metadata)
        return InsertResult(True, time.perf_counter() - t0, v.nbytes, False)

    def search(self, query, k: int, strategy: SearchStrategy = SearchStrategy.adaptive,
               filter: Callable[[str, Any], bool] | None = None) -> list[SearchResult]:
        if not self.ivf.trained:
            raise VSKError(-7, "IVF index is not trained")
        strategy = SearchStrategy(strategy)
        nprobe = (self.configuration.numberOfCentroids if strategy == SearchStrategy.exact
                  else self.configuration.numberOfProbes)
        q = np.ascontiguousarray(np.asarray(query, np.float32).reshape(1, -1))
        if k <= 0:
            return []
        want = min(k, MAX_K)
        k_try = want
        while True:
            dist, ids = self.ivf.search(q, k_try, nprobe=nprobe)  # vsk_ivf_search
            dist, ids = np.asarray(dist)[0], np.asarray(ids)[0]
            kept = []
            for dv, row in zip(dist.tolist(), ids.tolist()):
                if row < 0:
                    break
                if row in self._deleted:
                    continue
                if filter is not None and not filter(self._ids[row], self._meta[row]):
                    continue
                kept.append((dv, row))
            exhausted = bool((ids < 0).any())
            if len(kept) >= want or exhausted or k_try >= MAX_K:
                break
            k_try = min(2 * k_try, MAX_K)
        return [SearchResult(self._ids[row], float(dv), self._meta[row]) for dv, row in
                kept[:want]]

    def update(self, id: str, vector=None, metadata=None) -> bool:
        return False  # IVFIndex.update (:204-208)

    def delete(self, id: str) -> bool:
        row = self._row_of.pop(id, None)
        if row is None:
            return False
        self._deleted.add(row)
        return True

    def contains(self, id: str) -> bool:
        return id in self._row_of


class HIPIVFIndexingStrategy:
    """``IndexingStrategy`` whose ``createIndex()`` returns a ``HIPIVFIndex``
    (the HIP twin of IVFIndexingStrategy, API/Strategies/
    IndexingStrategies.swift:230-272)."""

    identifier = "ivf-hip"

    def __init__(self, accelerator: HIPAcceleratorStrategy, dimensions: int,
                 numClusters: int = 1024, nprobe: int = 16,
                 configuration: IVFConfiguration | None = None):
        self.accelerator = accelerator
        self.configuration = configuration or IVFConfiguration(
            dimensions=dimensions, numberOfCentroids=numClusters, numberOfProbes=nprobe)

    def createIndex(self) -> HIPIVFIndex:
        return HIPIVFIndex(self.accelerator, self.configuration)

"""Batched neighbour-distance evaluation for HNSW graph walks
(``vsk_hnsw_distances``), and a lockstep layer-0 search that uses it.

Reference: HNSWIndex (Indexes/HNSWIndex.swift of gifton/VectorStoreKit).
Its searchLayer0 (:1151-1212) and greedySearchLayer (:1035-1094) score each
unvisited neighbour of the visited node with DistanceComputer.distance
(:1920-1959), one call at a time.  Those distances do not depend on the
search state, so a node's neighbours can be scored together, and many
searches can be advanced in the same step: ``HNSWBatchSearch.search_layer0``
runs the reference's loop for every query on the host and hands all the
queries' neighbour lists of a step to one GPU launch.
"""
from __future__ import annotations

import numpy as np

from . import _lib
from ._lib import VSKError, as_buffer, out_buffer
from .engine import VectorDatabase

# DistanceComputer's metrics (euclidean, cosine without epsilon, manhattan);
# every other DistanceMetric falls back to euclidean (:1927-1937)
_HNSW_METRIC = {
    "euclidean": _lib.METRIC_L2,
    "cosine": _lib.METRIC_COSINE_NOEPS,
    "manhattan": _lib.METRIC_L1,
    "euclideanSquared": _lib.METRIC_L2SQ,
}


def hnsw_metric_code(metric) -> int:
    if isinstance(metric, int):
        return metric
    return _HNSW_METRIC.get(str(metric), _lib.METRIC_L2)


def neighbor_distances(db: VectorDatabase, queries, offsets, rows, metric="euclidean"):
    """out[j] = DistanceComputer.distance(query i, row rows[j]) for j in
    offsets[i]:offsets[i+1] (CSR), one launch for all queries."""
    ctx = db.ctx
    nq = int(queries.shape[0])
    qp, qk = as_buffer(queries, np.float32, (nq, db.d))
    op, ok = as_buffer(offsets, np.int64, (nq + 1,))
    total = int(offsets[-1])
    if total == 0:
        return np.empty(0, np.float32)
    rp, rk = as_buffer(rows, np.int32, (total,))
    outp, out = out_buffer((total,), np.float32, queries)
    ctx.check(ctx.lib.vsk_hnsw_distances(ctx.handle, db.handle, qp, nq, op, rp,
                                         hnsw_metric_code(metric), outp))
    return out


class HNSWBatchSearch:
    """searchLayer0 for a batch of queries in lockstep over one graph layer.

    ``adjacency[node]`` lists the node's layer-0 connections; ``deleted``
    nodes are skipped as ``isDeleted`` nodes are.  Per step every active
    query visits its closest candidate; the unvisited neighbours of all
    visited nodes are scored in one ``vsk_hnsw_distances`` call and then
    processed in neighbour order exactly as the reference's loop does, so
    each query's result equals the sequential search's."""

    def __init__(self, db: VectorDatabase, adjacency, metric="euclidean", deleted=()):
        self.db = db
        self.adjacency = adjacency
        self.metric = metric
        self.deleted = set(deleted)
        self.steps = 0
        self.launches = 0

    def search_layer0(self, queries, entries, ef: int):
        q = np.ascontiguousarray(np.asarray(queries, np.float32))
        nq = q.shape[0]
        if len(entries) != nq:
            raise VSKError(-4, "one entry point per query")
        for e in entries:
            if e in self.deleted:
                raise VSKError(-2, "Invalid entry point for layer 0")
        # the entry points' distances
        off = np.arange(nq + 1, dtype=np.int64)
        d0 = neighbor_distances(self.db, q, off, np.asarray(entries, np.int32), self.metric)
        self.launches += 1
        visited = [{int(e)} for e in entries]
        cand = [[(float(d0[i]), int(entries[i]))] for i in range(nq)]
        w = [[(float(d0[i]), int(entries[i]))] for i in range(nq)]
        active = list(range(nq))
        while active:
            self.steps += 1
            # each active query visits its closest candidate
            lists, still = [], []
            for i in active:
                if not cand[i]:
                    continue
                cand[i].sort(key=lambda t: t[0])
                cur = cand[i].pop(0)
                if len(w[i]) >= ef:
                    w[i].sort(key=lambda t: t[0], reverse=True)
                    if cur[0] > w[i][0][0]:
                        continue
                still.append(i)
                nbs = []
                if cur[1] not in self.deleted:
                    for nb in self.adjacency[cur[1]]:
                        if nb in visited[i]:
                            continue
                        visited[i].add(nb)
                        if nb not in self.deleted:
                            nbs.append(int(nb))
                lists.append(nbs)
            active = still
            if not active:
                break
            counts = np.array([len(x) for x in lists], np.int64)
            off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
            if off[-1] > 0:
                rows = np.concatenate([np.asarray(x, np.int32) for x in lists if x])
                dist = np.asarray(neighbor_distances(self.db, q[active], off, rows, self.metric))
                self.launches += 1
            for slot, i in enumerate(active):
                for j in range(off[slot], off[slot + 1]):
                    dv, nb = float(dist[j]), int(rows[j])
                    if len(w[i]) < ef:
                        cand[i].append((dv, nb))
                        w[i].append((dv, nb))
                    else:
                        w[i].sort(key=lambda t: t[0], reverse=True)
                        if dv < w[i][0][0]:
                            cand[i].append((dv, nb))
                            w[i][0] = (dv, nb)
        for i in range(nq):
            w[i].sort(key=lambda t: t[0])
        return w

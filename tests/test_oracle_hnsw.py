"""The oracle's HNSW distances (DistanceComputer, Indexes/HNSWIndex.swift:
1920-1959) and searchLayer0 restatement, pinned without the reference:
numpy fp32 left folds, closed forms (orthogonal cosine 1, parallel 0,
opposite 2, zero vector NaN since there is no epsilon), and brute force."""
import numpy as np

from oracle import oracle as O


def test_hnsw_distance_folds_and_kats():
    rng = np.random.default_rng(1)
    for d in (1, 7, 128, 300):
        q = rng.standard_normal(d).astype(np.float32)
        x = rng.standard_normal(d).astype(np.float32)
        diff = (q - x).astype(np.float32)
        l2sq = np.cumsum(diff * diff, dtype=np.float32)[-1]
        assert O.hnsw_distance(q, x, O.L2SQ) == l2sq
        assert O.hnsw_distance(q, x, O.L2) == np.sqrt(l2sq, dtype=np.float32)
        l1 = np.cumsum(np.abs(diff), dtype=np.float32)[-1]
        assert O.hnsw_distance(q, x, O.L1) == l1
        dot = np.cumsum(q * x, dtype=np.float32)[-1]
        m1 = np.sqrt(np.cumsum(q * q, dtype=np.float32)[-1], dtype=np.float32)
        m2 = np.sqrt(np.cumsum(x * x, dtype=np.float32)[-1], dtype=np.float32)
        want = np.float32(1) - dot / np.float32(m1 * m2)
        assert O.hnsw_distance(q, x, O.COSINE_NOEPS) == want
        assert abs(float(want) - (1 - float(q.astype(np.float64) @ x) /
                                  (np.linalg.norm(q.astype(np.float64)) *
                                   np.linalg.norm(x.astype(np.float64))))) < 1e-5
    e = np.eye(4, dtype=np.float32)
    assert O.hnsw_distance(e[0], e[1], O.L2) == np.float32(np.sqrt(2))
    assert O.hnsw_distance(e[0], e[1], O.COSINE_NOEPS) == 1.0
    v = np.array([3, 4, 0, 0], np.float32)
    assert O.hnsw_distance(v, v, O.COSINE_NOEPS) == 0.0
    assert O.hnsw_distance(v, -v, O.COSINE_NOEPS) == 2.0
    assert O.hnsw_distance(v, v, O.L2) == 0.0
    # no epsilon: a zero vector gives NaN, where the epsilon form gives 1
    z = np.zeros(4, np.float32)
    assert np.isnan(O.hnsw_distance(z, v, O.COSINE_NOEPS))
    assert O.distance(z, v, O.COSINE) == 1.0


def test_hnsw_distances_csr():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((500, 19)).astype(np.float32)
    q = rng.standard_normal((4, 19)).astype(np.float32)
    counts = [3, 0, 7, 2]
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    rows = rng.integers(0, 500, off[-1]).astype(np.int32)
    out = O.hnsw_distances(q, x, off, rows, O.L1)
    for i in range(4):
        for j in range(off[i], off[i + 1]):
            assert out[j] == O.hnsw_distance(q[i], x[rows[j]], O.L1)


def test_search_layer0_complete_graph_is_brute_force():
    """On a complete graph with ef >= n the walk visits every node: the
    result is every node, sorted by distance (ties by visiting order)."""
    rng = np.random.default_rng(3)
    n = 40
    x = rng.standard_normal((n, 8)).astype(np.float32)
    q = rng.standard_normal(8).astype(np.float32)
    adj = [[j for j in range(n) if j != i] for i in range(n)]
    res = O.search_layer0(q, x, adj, 5, n, O.L2)
    d = np.array([O.hnsw_distance(q, x[i], O.L2) for i in range(n)], np.float32)
    assert [t[1] for t in res] == list(np.argsort(d, kind="stable"))
    # ef smaller than n: the ef nearest of a complete graph
    res = O.search_layer0(q, x, adj, 5, 10, O.L2)
    assert sorted(t[1] for t in res) == sorted(np.argsort(d, kind="stable")[:10])

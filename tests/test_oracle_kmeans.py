"""Pins the CPU oracle's k-means restatement (oracle/vsk_oracle.c,
vsko_kmeans_cluster and its seeding) against closed forms, library routines
and invariants, not against a retyped copy of its own loops.

Reference: Clustering/KMeansClustering.swift (cluster :48-113, random init
:197-207, k-means++ :209-259, assignment :271-295, update :342-380,
SeedableRNG :480-491) and its test NewIndexTests.swift:12-57.
"""
import numpy as np
import pytest

from oracle import oracle as O

A, C = 2862933555777941757, 3037000493
M64 = (1 << 64) - 1
GOLDEN = 0x9E3779B97F4A7C15


def lcg(s):
    return (s * A + C) & M64


def test_lcg_and_bounded_power_of_two():
    """For bound = 2^b, Lemire's draw is the top b bits of the LCG output
    (the rejection branch needs the low 64 - b bits of r all zero)."""
    for seed in [0, 1, 42, 2**63 + 5, M64]:
        for b in [1, 7, 20, 33]:
            v, st = O.swift_bounded(seed, 1 << b)
            r = lcg(seed)
            assert st == r
            assert v == r >> (64 - b)


def test_bounded_uniform():
    """Int.random(in: 0..<10) over a chain of draws is uniform (chi-square)."""
    st, counts = 12345, np.zeros(10)
    for _ in range(20000):
        v, st = O.swift_bounded(st, 10)
        assert 0 <= v < 10
        counts[v] += 1
    chi2 = ((counts - 2000.0) ** 2 / 2000.0).sum()
    assert chi2 < 30.0  # 9 dof, p ~ 5e-4


def test_init_random_shuffle_prefix():
    """Fisher-Yates from the front: rows[0] is the first bounded draw over n;
    k = n gives a permutation; picks are distinct; rows[0] is uniform over
    seeds."""
    for seed in range(20):
        v, _ = O.swift_bounded(seed, 50)
        rows = O.kmeans_init_random(50, 7, seed)
        assert rows[0] == v
        assert len(set(rows.tolist())) == 7 and rows.min() >= 0 and rows.max() < 50
    assert sorted(O.kmeans_init_random(31, 31, 9).tolist()) == list(range(31))
    counts = np.bincount([O.kmeans_init_random(8, 3, s)[0] for s in range(8000)], minlength=8)
    chi2 = ((counts - 1000.0) ** 2 / 1000.0).sum()
    assert chi2 < 25.0


def _seq_l2(x, c):
    """sqrt of the fp32 sum of squared differences in dimension order
    (np.cumsum is sequential by definition)."""
    t = (x - c).astype(np.float32)
    return np.sqrt(np.cumsum(t * t, axis=-1, dtype=np.float32)[..., -1])


def test_k1_mean_inertia_and_convergence():
    """k = 1: the centroid is the fp32 row-order sum / n.  Iteration 1 runs
    from a sampled row and cannot converge (previous = +inf), iteration 2
    from the mean, iteration 3 repeats it exactly and stops; the inertia is
    the fp32 row-order sum of the sqrt distances to the mean."""
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((3001, 13)) * 3 + 1).astype(np.float32)
    c, a, it, conv, inertia = O.kmeans_cluster(x, 1, seed=4)
    mean = np.cumsum(x, axis=0, dtype=np.float32)[-1] / np.float32(x.shape[0])
    np.testing.assert_array_equal(c[0], mean)
    assert (a == 0).all() and it == 3 and conv
    dist = _seq_l2(x, mean)
    assert inertia == np.cumsum(dist, dtype=np.float32)[-1]
    # a float64 mean rounded once differs: the fp32 row order is what is pinned
    assert (x.astype(np.float64).mean(axis=0).astype(np.float32) != mean).any()


def test_separated_clusters_custom_init():
    """Tight, far-apart clusters from their true centres: assignments are the
    labels, centroids the per-cluster fp32 row-order means; iteration 2 runs
    from the means, iteration 3 repeats it and stops."""
    rng = np.random.default_rng(2)
    k, d, n = 6, 9, 1200
    centres = (rng.standard_normal((k, d)) * 50).astype(np.float32)
    lab = rng.integers(0, k, n)
    x = (centres[lab] + rng.standard_normal((n, d))).astype(np.float32)
    c, a, it, conv, _ = O.kmeans_cluster(x, k, init_method="custom", init=centres)
    np.testing.assert_array_equal(a, lab)
    for j in range(k):
        rows = x[lab == j]
        np.testing.assert_array_equal(
            c[j], np.cumsum(rows, axis=0, dtype=np.float32)[-1] / np.float32(len(rows)))
    assert it == 3 and conv


def test_first_assignment_is_float64_argmin():
    """max_iter = 1 from given centroids: each row goes to the float64 nearest
    centroid (rows with a near tie are skipped); ties go to the lower index."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4000, 24)).astype(np.float32)
    init = rng.standard_normal((37, 24)).astype(np.float32)
    _, a, it, conv, _ = O.kmeans_cluster(x, 37, init_method="custom", init=init, max_iter=1)
    d64 = ((x[:, None, :].astype(np.float64) - init[None].astype(np.float64)) ** 2).sum(-1)
    srt = np.sort(d64, axis=1)
    clear = srt[:, 1] - srt[:, 0] > 1e-4 * srt[:, 0]
    np.testing.assert_array_equal(a[clear], d64.argmin(axis=1)[clear])
    assert it == 1 and not conv
    # an exact duplicate centroid: the first index wins
    init2 = np.concatenate([init[:1], init[:1]])
    _, a2, _, _, _ = O.kmeans_cluster(x, 2, init_method="custom", init=init2, max_iter=1)
    assert (a2 == 0).all()


def test_weights():
    """Weights 2.0 scale sums and counts exactly: same result as none.  A
    cluster whose weight sum is 0 is refilled like an empty one."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((900, 6)).astype(np.float32)
    ref = O.kmeans_cluster(x, 5, seed=8, max_iter=7)
    w2 = O.kmeans_cluster(x, 5, seed=8, max_iter=7, weights=np.full(900, 2.0, np.float32))
    np.testing.assert_array_equal(ref[0], w2[0])
    np.testing.assert_array_equal(ref[1], w2[1])
    init = np.stack([x[:450].mean(0), x[450:].mean(0) + 100]).astype(np.float32)
    w = np.ones(900, np.float32)
    c, a, _, _, _ = O.kmeans_cluster(x, 2, init_method="custom", init=init, max_iter=1,
                                     weights=w, seed=11)
    r, _ = O.swift_bounded((11 + GOLDEN) & M64, 900)
    assert (a == 0).all()
    np.testing.assert_array_equal(c[1], x[r])


def test_empty_cluster_refill_and_zero_iterations():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((500, 4)).astype(np.float32)
    init = np.stack([np.zeros(4), np.full(4, 1e3), np.full(4, -1e3)]).astype(np.float32)
    c, a, it, conv, _ = O.kmeans_cluster(x, 3, init_method="custom", init=init, max_iter=1,
                                         seed=21)
    st = (21 + GOLDEN) & M64
    r1, st = O.swift_bounded(st, 500)
    r2, st = O.swift_bounded(st, 500)
    np.testing.assert_array_equal(c[1], x[r1])  # ascending cluster order
    np.testing.assert_array_equal(c[2], x[r2])
    c0, a0, it0, conv0, in0 = O.kmeans_cluster(x, 3, init_method="custom", init=init,
                                               max_iter=0)
    np.testing.assert_array_equal(c0, init)
    assert (a0 == 0).all() and it0 == 0 and not conv0 and np.isinf(in0)


def test_reference_test_properties():
    """NewIndexTests.swift:12-31 (100 x 8, k = 5) and :33-57 (random /
    k-means++ / custom init on 50 x 4, k = 3)."""
    rng = np.random.default_rng(7)
    v = rng.random((100, 8), dtype=np.float32)
    c, a, it, conv, inertia = O.kmeans_cluster(v, 5, init_method="kMeansPlusPlus", seed=1)
    assert c.shape == (5, 8) and a.shape == (100,)
    assert conv or it > 0
    assert inertia > 0 and a.min() >= 0 and a.max() < 5
    v = rng.random((50, 4), dtype=np.float32)
    for m in ["random", "kMeansPlusPlus"]:
        assert O.kmeans_cluster(v, 3, init_method=m, seed=42)[0].shape == (3, 4)
    cust = np.stack([v[0], v[10], v[20]])
    assert O.kmeans_cluster(v, 3, init_method="custom", init=cust)[0].shape == (3, 4)


def test_plusplus_d2_law_and_degenerate():
    """Points 0, 1, 2, 4 on a line.  Given the first pick at 0, the second is
    1, 2 or 4 with probability 1:4:16 (D^2), not 1:2:4 (D) -- over many
    seeds (all picks come from one stream, so the second draw is not tied to
    the first).  Identical rows are degenerate data."""
    x = np.array([[0.0], [1.0], [2.0], [4.0]], np.float32)
    counts = np.zeros(4)
    for s in range(40000):
        rows = O.kmeans_init_plusplus(x, 2, s)
        if rows[0] == 0:
            counts[rows[1]] += 1
    assert counts[0] == 0
    tot = counts.sum()
    expect = tot * np.array([1.0, 4.0, 16.0]) / 21.0
    chi2 = ((counts[1:] - expect) ** 2 / expect).sum()
    assert tot > 5000 and chi2 < 15.0
    for s in range(30):
        rows = O.kmeans_init_plusplus(np.random.default_rng(s).random((40, 3), np.float32), 12, s)
        assert len(set(rows.tolist())) == 12
        assert rows[0] == O.swift_bounded(s, 40)[0]
    with pytest.raises(ValueError):
        O.kmeans_cluster(np.ones((10, 3), np.float32), 2, init_method="kMeansPlusPlus")

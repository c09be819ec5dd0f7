"""k-means on the GPU (vsk_kmeans) against the CPU oracle's restatement of
KMeansClustering.cluster (Clustering/KMeansClustering.swift:48-113).  Every
part is bit-exact: assignments (strict '<' on sequential sqrt-L2),
centroids (fp32 row-order sums, fp32 division), inertia (fp32 row-order
sum), iteration count and converged flag, and the seeding (Swift shuffle
prefix, k-means++ with exact fixed-point D^2 weights)."""
import numpy as np
import pytest

from oracle import oracle as O
from vectorstorekit_amd import (IVFConfiguration, IVFIndex, KMeansClustering,
                                KMeansClusteringConfiguration, ProductQuantizer, VSKError)

pytestmark = pytest.mark.gpu


def _mixture(seed, n, d, ncent, spread=4.0):
    rng = np.random.default_rng(seed)
    cent = rng.standard_normal((ncent, d)).astype(np.float32) * spread
    lab = rng.integers(0, ncent, n)
    return (cent[lab] + rng.standard_normal((n, d)).astype(np.float32)).astype(np.float32)


def _check(res, ref):
    c, a, it, conv, inertia = ref
    np.testing.assert_array_equal(np.asarray(res.assignments), a)
    np.testing.assert_array_equal(np.asarray(res.centroids), c)
    assert res.iterations == it and res.converged == conv
    assert np.float32(res.inertia) == inertia or (np.isinf(inertia) and np.isinf(res.inertia))


@pytest.mark.parametrize("method", ["random", "kMeansPlusPlus"])
@pytest.mark.parametrize("shape", [(3000, 16, 8), (5000, 37, 17), (2500, 128, 300),
                                   (700, 5, 1), (4000, 8, 256), (1200, 64, 1200)])
def test_kmeans_bit_exact(ctx, method, shape):
    """Ragged and padded dimensions (5, 37), one to three radix passes
    (k = 1, 8, 17, 256, 300, 1200), k = n (every row its own cluster)."""
    n, d, k = shape
    print(f"kmeans {method} n={n} d={d} k={k}", flush=True)
    x = _mixture(n + d + k, n, d, max(2, k // 2))
    cfg = KMeansClusteringConfiguration(maxIterations=12, tolerance=1e-4, initMethod=method,
                                        seed=n + k)
    res = KMeansClustering(ctx, cfg).cluster(x, k)
    ref = O.kmeans_cluster(x, k, init_method=method, max_iter=12, tol=1e-4, seed=n + k)
    _check(res, ref)


def test_kmeans_custom_weights_empty_clusters(ctx):
    """Custom start with centroids far from the data (empty clusters refilled
    from the seeded stream), weights, and a run to convergence."""
    x = _mixture(9, 6000, 24, 10)
    rng = np.random.default_rng(4)
    init = np.concatenate([x[:6], np.full((4, 24), 1e4, np.float32)]).astype(np.float32)
    w = rng.random(6000, dtype=np.float32) * 3
    for weights in (None, w):
        cfg = KMeansClusteringConfiguration(maxIterations=60, tolerance=1e-3, initMethod="custom",
                                            seed=77, customCentroids=init)
        res = KMeansClustering(ctx, cfg).cluster(x, 10, weights=weights)
        ref = O.kmeans_cluster(x, 10, init_method="custom", init=init, weights=weights,
                               max_iter=60, tol=1e-3, seed=77)
        _check(res, ref)
    cfg = KMeansClusteringConfiguration(maxIterations=0, initMethod="custom", customCentroids=init)
    res = KMeansClustering(ctx, cfg).cluster(x, 10)
    _check(res, O.kmeans_cluster(x, 10, init_method="custom", init=init, max_iter=0))


def test_kmeans_device_tensors(ctx):
    import torch

    x = _mixture(12, 20_000, 32, 64)
    xt = torch.from_numpy(x).cuda()
    cfg = KMeansClusteringConfiguration(maxIterations=5, initMethod="random", seed=3)
    res = KMeansClustering(ctx, cfg).cluster(xt, 64)
    assert res.centroids.is_cuda and res.assignments.is_cuda
    ref = O.kmeans_cluster(x, 64, init_method="random", max_iter=5, seed=3)
    np.testing.assert_array_equal(res.centroids.cpu().numpy(), ref[0])
    np.testing.assert_array_equal(res.assignments.cpu().numpy(), ref[1])


def test_kmeans_errors(ctx):
    x = np.ones((10, 3), np.float32)
    with pytest.raises(VSKError) as e:
        KMeansClustering(ctx, KMeansClusteringConfiguration(seed=1)).cluster(x, 2)
    assert e.value.kind == "invalidArgument" and "degenerate" in str(e.value)
    with pytest.raises(VSKError) as e:
        KMeansClustering(ctx, KMeansClusteringConfiguration(seed=1)).cluster(x, 11)
    assert e.value.kind == "invalidArgument"
    with pytest.raises(VSKError) as e:
        KMeansClustering(ctx).cluster(np.zeros((0, 3), np.float32), 1)
    assert e.value.kind == "emptyInput"
    # the context still works after the errors
    r = KMeansClustering(ctx, KMeansClusteringConfiguration(initMethod="random", seed=2)).cluster(
        _mixture(1, 100, 3, 4), 4)
    assert r.iterations > 0


def test_ivf_train_uses_kmeans(ctx):
    """IVFIndex.train(on:) runs clusteringConfig's k-means; the index then
    searches exactly like one built from those centroids."""
    x = _mixture(21, 8000, 16, 32)
    cfg = KMeansClusteringConfiguration(maxIterations=20, initMethod="kMeansPlusPlus", seed=5)
    idx = IVFIndex(ctx, IVFConfiguration(dimensions=16, numberOfCentroids=32, numberOfProbes=4,
                                         clusteringConfig=cfg))
    res = idx.train(x)
    ref = O.kmeans_cluster(x, 32, init_method="kMeansPlusPlus", max_iter=20, seed=5)
    np.testing.assert_array_equal(idx.getCentroids(), ref[0])
    assert res.iterations == ref[2]
    idx.insert(x)
    q = x[:50] + 0.01
    d, i = idx.search(q, 5)
    od, oi = O.ivf_search(q, x, np.arange(8000, dtype=np.int64), O.ivf_assign(x, ref[0]),
                          ref[0], 4, 5)
    np.testing.assert_array_equal(i, oi)
    np.testing.assert_array_equal(d, od)


def test_pq_train_uses_kmeans(ctx):
    """ProductQuantizer.train: per segment m, k-means++ seeded with m,
    tolerance 1e-4 (ProductQuantizer.swift:270-324)."""
    x = _mixture(3, 4000, 32, 20)
    pq = ProductQuantizer.train(ctx, x, 4, 16, iterations=6)
    for m in range(4):
        seg = np.ascontiguousarray(x[:, m * 8:(m + 1) * 8])
        ref = O.kmeans_cluster(seg, 16, init_method="kMeansPlusPlus", max_iter=6, tol=1e-4,
                               seed=m)
        np.testing.assert_array_equal(pq.codebooks[m], ref[0])


def test_kmeans_config3_scale(ctx):
    """IVF training at config 3's scale: 1M x 128 rows of a 4,096-Gaussian
    mixture, nlist 4096, one iteration from the jittered true centres.
    Checked by properties the oracle can afford at this size: a row sample's
    assignments equal the oracle's argmin against the starting centroids, a
    sample of clusters' centroids equals the fp32 row-order mean of their
    rows bit for bit, and the inertia equals the fp32 row-order sum of all
    rows' sequential sqrt-L2 distances to their assigned starting centroid."""
    import torch

    n, d, ncent = 1_000_000, 128, 4096
    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    cent = 2.0 * torch.randn(ncent, d, generator=g, device="cuda")
    g.manual_seed(5)
    a = torch.randint(0, ncent, (n,), generator=g, device="cuda")
    g.manual_seed(1)
    x = cent[a] + 0.5 * torch.randn(n, d, generator=g, device="cuda")
    g.manual_seed(4)
    c0 = cent + 0.1 * torch.randn(ncent, d, generator=g, device="cuda")
    print("kmeans config3 scale 1Mx128 k4096 max_iter 1", flush=True)
    cfg = KMeansClusteringConfiguration(maxIterations=1, initMethod="custom", customCentroids=c0)
    res = KMeansClustering(ctx, cfg).cluster(x, ncent)
    xh, c0h = x.cpu().numpy(), c0.cpu().numpy()
    assign = res.assignments.cpu().numpy()
    cen = res.centroids.cpu().numpy()
    sample = np.random.default_rng(0).choice(n, 20_000, replace=False)
    np.testing.assert_array_equal(assign[sample], O.ivf_assign(xh[sample], c0h))
    for cl in np.random.default_rng(1).choice(ncent, 64, replace=False):
        rows = xh[assign == cl]
        if len(rows) == 0:
            continue
        mean = np.cumsum(rows, axis=0, dtype=np.float32)[-1] / np.float32(len(rows))
        np.testing.assert_array_equal(cen[cl], mean)
    dist = np.empty(n, np.float32)
    for r in range(0, n, 100_000):
        t = xh[r:r + 100_000] - c0h[assign[r:r + 100_000]]
        dist[r:r + 100_000] = np.sqrt(np.cumsum(t * t, axis=1, dtype=np.float32)[:, -1])
    assert res.iterations == 1 and not res.converged
    assert np.float32(res.inertia) == np.cumsum(dist, dtype=np.float32)[-1]


@pytest.fixture(scope="module")
def screen_ctx():
    """A context whose argmin takes the bf16 screen at every size."""
    import os

    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from vectorstorekit_amd import Context

    old = os.environ.get("VSK_FLAT_KERNEL")
    os.environ["VSK_FLAT_KERNEL"] = "screen"
    try:
        c = Context(0)
    finally:
        if old is None:
            del os.environ["VSK_FLAT_KERNEL"]
        else:
            os.environ["VSK_FLAT_KERNEL"] = old
    yield c
    c.close()


@pytest.mark.parametrize("method", ["random", "kMeansPlusPlus"])
@pytest.mark.parametrize("shape", [(5000, 37, 17), (2500, 128, 300), (1200, 64, 1200),
                                   (20_000, 96, 64), (3001, 200, 257)])
def test_kmeans_screen_bit_exact(screen_ctx, method, shape):
    """The screened assignment (bf16 MFMA top-2, bound test, exact winner)
    gives the oracle's k-means bit for bit: partial row and query tiles
    (k = 17, 257, 300; n = 3001), padded dimensions (37 -> 64, 200 -> 256)."""
    n, d, k = shape
    print(f"kmeans screen {method} n={n} d={d} k={k}", flush=True)
    x = _mixture(n * 3 + d + k, n, d, max(2, k // 2))
    cfg = KMeansClusteringConfiguration(maxIterations=8, tolerance=1e-4, initMethod=method,
                                        seed=n + 3 * k)
    res = KMeansClustering(screen_ctx, cfg).cluster(x, k)
    ref = O.kmeans_cluster(x, k, init_method=method, max_iter=8, tol=1e-4, seed=n + 3 * k)
    _check(res, ref)


def test_screen_argmin_ties_fall_back(screen_ctx):
    """Duplicated centroids tie every row near them: the screen cannot
    decide, the collecting pass rescores the tied rows exactly and the first
    duplicate wins.  81 copies of one centroid overflow the 64-candidate
    lists: those rows take the exact scan over every centroid."""
    rng = np.random.default_rng(8)
    d = 64
    base = (rng.standard_normal((300, d)) * 3).astype(np.float32)
    # rows 300..349 duplicate 0..49; rows 350..429 copy row 299
    cent = np.concatenate([base, base[:50], np.repeat(base[299:300], 80, axis=0)])
    cent = cent.astype(np.float32)
    x = (base[rng.integers(0, 300, 30_000)] + rng.standard_normal((30_000, d))).astype(np.float32)
    idx = IVFIndex(screen_ctx, IVFConfiguration(dimensions=d, numberOfCentroids=len(cent),
                                                numberOfProbes=4))
    idx.set_centroids(cent)
    got = idx.assign(x)
    np.testing.assert_array_equal(got, O.ivf_assign(x, cent))
    assert (got < 300).all()
    screen_ctx.profile(True)
    screen_ctx.profile_reset()
    idx.assign(x)
    stats = screen_ctx.profile_stats()
    screen_ctx.profile(False)
    for key in ("flat_screen_top2", "screen_argmin_collect", "screen_argmin_fallback"):
        assert key in stats, key

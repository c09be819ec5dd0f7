"""IVF-Flat on the GPU against the oracle.  Probing, assignment and the list
scan sum every squared difference in the reference's order without FMA, so
probes, assignments, distances and ids must be bit-identical."""
import json
import os

import numpy as np
import pytest

from oracle import oracle as O
from parity import assert_sorted_unique, recall
from vectorstorekit_amd import (IVFConfiguration, IVFIndex, KMeansClusteringConfiguration,
                                VSKError)

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _mixture(seed, ncent, n, d, nq):
    rng = np.random.default_rng(seed)
    cent = (2.0 * rng.standard_normal((ncent, d))).astype(np.float32)
    a = rng.integers(0, ncent, n)
    x = (cent[a] + 0.5 * rng.standard_normal((n, d))).astype(np.float32)
    qa = rng.integers(0, ncent, nq)
    q = (cent[qa] + 0.5 * rng.standard_normal((nq, d))).astype(np.float32)
    c = (cent + 0.1 * rng.standard_normal(cent.shape)).astype(np.float32)
    return x, q, c


def _index(ctx, c, x, ids=None, nprobe=8):
    idx = IVFIndex(ctx, IVFConfiguration(dimensions=c.shape[1], numberOfCentroids=c.shape[0],
                                         numberOfProbes=nprobe))
    idx.set_centroids(c)
    if x is not None:
        idx.insert(x, ids)
    return idx


@pytest.mark.parametrize("shape", [(64, 20_000, 128, 200, 8, 10), (37, 5000, 33, 50, 5, 7),
                                   (16, 3000, 24, 40, 16, 20)])
def test_ivf_bit_exact(ctx, shape):
    ncent, n, d, nq, nprobe, k = shape
    print(f"ivf ncent={ncent} n={n} d={d} nq={nq} nprobe={nprobe} k={k}", flush=True)
    x, q, c = _mixture(ncent + n, ncent, n, d, nq)
    ids = np.arange(n, dtype=np.int64) * 3 + 7
    idx = _index(ctx, c, x, ids, nprobe)
    lists = O.ivf_assign(x, c)
    np.testing.assert_array_equal(idx.assign(x), lists)
    np.testing.assert_array_equal(idx.list_sizes(), np.bincount(lists, minlength=ncent))
    np.testing.assert_array_equal(idx.probe(q, nprobe), O.ivf_probe(q, c, nprobe))
    gd, gi = idx.search(q, k)
    od, oi = O.ivf_search(q, x, ids, lists, c, nprobe, k)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)


def _screen_ctx():
    """A context whose list scans always take the bf16 screen."""
    from vectorstorekit_amd import Context

    old = os.environ.get("VSK_FLAT_KERNEL")
    os.environ["VSK_FLAT_KERNEL"] = "screen"
    try:
        sctx = Context(0)
    finally:
        if old is None:
            del os.environ["VSK_FLAT_KERNEL"]
        else:
            os.environ["VSK_FLAT_KERNEL"] = old
    sctx.profile(True)
    return sctx


@pytest.mark.parametrize("shape", [(64, 20_000, 128, 200, 8, 10, "euclidean"),
                                   (37, 5000, 33, 150, 5, 7, "euclideanSquared"),
                                   (40, 12_000, 160, 90, 40, 100, "euclidean"),
                                   (24, 9000, 256, 70, 6, 64, "euclideanSquared"),
                                   (16, 3000, 24, 40, 16, 20, "euclidean"),
                                   (32, 15_000, 64, 30, 12, 300, "euclidean")])
def test_ivf_screen_bit_exact(shape):
    """The list scan through the bf16 screen (forced at these sizes): query
    groups of up to 64 per list, the screened keys within the bound's margin
    of the k-th, their exact rescore.  Plane widths of 2, 4, 6 and 8 k-steps,
    both euclidean metrics, k above 64 and above 256 (where the margin,
    rescore and selections are launches of their own rather than one fused
    tail), every list probed; then rows added (the plane is made again),
    among them a block of identical rows, more than the margin's slots hold
    (1,024, or 4k above k = 256), so the queries next to it have their whole
    candidate set rescored.  Bit-exact against the oracle."""
    ncent, n, d, nq, nprobe, k, metric = shape
    print(f"ivf screen ncent={ncent} n={n} d={d} nq={nq} nprobe={nprobe} k={k} {metric}",
          flush=True)
    sq = metric == "euclideanSquared"
    x, q, c = _mixture(ncent + n + 1, ncent, n, d, nq)
    ids = np.arange(n, dtype=np.int64) * 3 + 7
    sctx = _screen_ctx()
    idx = _index(sctx, c, x, ids, nprobe)
    lists = O.ivf_assign(x, c)
    np.testing.assert_array_equal(idx.probe(q, nprobe), O.ivf_probe(q, c, nprobe))
    gd, gi = idx.search(q, k, metric=metric)
    assert "ivf_list_screen" in sctx.profile_stats(), "the screen did not run"
    assert "ivf_probe_screen" in sctx.profile_stats(), "the probe's screen did not run"
    od, oi = O.ivf_search(q, x, ids, lists, c, nprobe, k, squared=sq)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd.view(np.uint32), od.view(np.uint32))
    # rows added after the plane was made, among them 1,100 copies of one
    # row next to the first query
    rng = np.random.default_rng(n)
    ndup = max(1100, 4 * k + 100)
    dup = np.repeat(q[:1] + 0.01 * rng.standard_normal((1, d)).astype(np.float32), ndup, 0)
    extra = np.concatenate([x[:1000] + 0.1, dup]).astype(np.float32)
    eids = np.arange(n, n + len(extra), dtype=np.int64) * 3 + 7
    idx.insert(extra, eids)
    x2 = np.concatenate([x, extra])
    ids2 = np.concatenate([ids, eids])
    lists2 = O.ivf_assign(x2, c)
    fallback = "ivf_screen_tail" if k <= 256 else "ivf_screen_redo"
    before = sctx.profile_stats().get(fallback, (0, 0.0, 0.0))[2]
    gd, gi = idx.search(q, k, metric=metric)
    od, oi = O.ivf_search(q, x2, ids2, lists2, c, nprobe, k, squared=sq)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd.view(np.uint32), od.view(np.uint32))
    # the fallback's work count is the number of queries that overflowed
    assert sctx.profile_stats()[fallback][2] > before, "no query overflowed"
    sctx.close()


def test_ivf_probe_screen_overflow():
    """The probe through the screen when more centroids than its margin
    slots (1,024) tie with the nprobe-th: 1,100 copies of one centroid next
    to the queries.  Those queries have every centroid's exact distance
    ranked instead; probes (ties by centroid index) and results bit-exact
    against the oracle."""
    rng = np.random.default_rng(5)
    d, n, nq, nprobe, k = 32, 6000, 40, 8, 10
    base = rng.standard_normal((100, d)).astype(np.float32) * 3
    q = (base[0] + 0.3 * rng.standard_normal((nq, d))).astype(np.float32)
    c = np.concatenate([base, np.repeat(base[:1] + 0.05, 1100, 0)]).astype(np.float32)
    x = (base[rng.integers(0, 100, n)] + 0.3 * rng.standard_normal((n, d))).astype(np.float32)
    sctx = _screen_ctx()
    idx = _index(sctx, c, x, None, nprobe)
    np.testing.assert_array_equal(idx.probe(q, nprobe), O.ivf_probe(q, c, nprobe))
    # the fallback's work count is the number of queries that overflowed
    assert sctx.profile_stats()["ivf_probe_tail"][2] > 0
    lists = O.ivf_assign(x, c)
    gd, gi = idx.search(q, k)
    od, oi = O.ivf_search(q, x, np.arange(n, dtype=np.int64), lists, c, nprobe, k)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd.view(np.uint32), od.view(np.uint32))
    sctx.close()


def test_ivf_screen_exact_strategy_many_lists():
    """The screened list scan when every one of more lists than a selection
    holds is probed (the .exact strategy with 1,100 lists: probes in index
    order, candidate segments of every row), for both euclidean metrics;
    bit-exact against the oracle."""
    x, q, c = _mixture(21, 1100, 9000, 24, 30)
    sctx = _screen_ctx()
    idx = _index(sctx, c, x, None, 8)
    lists = O.ivf_assign(x, c)
    ids = np.arange(len(x), dtype=np.int64)
    for metric in ("euclidean", "euclideanSquared"):
        print(f"ivf screen exact strategy, 1100 lists, {metric}", flush=True)
        gd, gi = idx.search(q, 12, strategy="exact", metric=metric)
        od, oi = O.ivf_search(q, x, ids, lists, c, 1100, 12, squared=metric != "euclidean")
        np.testing.assert_array_equal(gi, oi)
        np.testing.assert_array_equal(gd.view(np.uint32), od.view(np.uint32))
    assert "ivf_list_screen" in sctx.profile_stats()
    sctx.close()


def test_ivf_screen_unclustered_bit_exact():
    """Rows without cluster structure (i.i.d. normal), many probes, so many
    candidates lie within the screen's margin of the k-th.  Bit-exact
    against the oracle, both euclidean metrics."""
    rng = np.random.default_rng(77)
    ncent, n, d, nq, nprobe, k = 64, 20_000, 48, 120, 24, 10
    x = rng.standard_normal((n, d)).astype(np.float32)
    q = rng.standard_normal((nq, d)).astype(np.float32)
    c = rng.standard_normal((ncent, d)).astype(np.float32)
    sctx = _screen_ctx()
    idx = _index(sctx, c, x, None, nprobe)
    lists = O.ivf_assign(x, c)
    ids = np.arange(n, dtype=np.int64)
    for metric in ("euclidean", "euclideanSquared"):
        print(f"ivf screen unclustered {metric}", flush=True)
        gd, gi = idx.search(q, k, metric=metric)
        od, oi = O.ivf_search(q, x, ids, lists, c, nprobe, k, squared=metric != "euclidean")
        np.testing.assert_array_equal(gi, oi)
        np.testing.assert_array_equal(gd.view(np.uint32), od.view(np.uint32))
    assert "ivf_list_screen" in sctx.profile_stats()
    sctx.close()


def _screen_ctx_keep_all():
    """A screen context whose list scan keeps every candidate's word
    (VSK_IVF_COMPACT=0) instead of those under each query's bound."""
    old = os.environ.get("VSK_IVF_COMPACT")
    os.environ["VSK_IVF_COMPACT"] = "0"
    try:
        return _screen_ctx()
    finally:
        if old is None:
            del os.environ["VSK_IVF_COMPACT"]
        else:
            os.environ["VSK_IVF_COMPACT"] = old


@pytest.mark.parametrize("nprobe,k", [(6, 25), (2, 25), (12, 1), (8, 64), (100, 10),
                                     (20, 100)])
def test_ivf_screen_compact_bound(nprobe, k):
    """The screened list scan keeps only the candidates under each query's
    bound: the smallest d + R (centroid distance plus list radius) at which
    the probed lists hold k rows.  Lists of about 10 rows, so the bound
    comes from several lists (k = 25), from none (nprobe 2: fewer candidates
    than k, every one kept, results padded), k = 1 and k = 64 (the tail a
    wave per query), nprobe 100 and k = 100 (the tail a workgroup per
    query over the compact candidates); both euclidean metrics, then rows
    added (the radii are made again with the plane).  Bit-identical to the
    scan that keeps every candidate and to the oracle."""
    x, q, c = _mixture(31, 300, 3000, 32, 60)
    ids = np.arange(len(x), dtype=np.int64) * 2 + 1
    sctx, actx = _screen_ctx(), _screen_ctx_keep_all()
    a, b = _index(sctx, c, x, ids, nprobe), _index(actx, c, x, ids, nprobe)
    lists = O.ivf_assign(x, c)
    for step in range(2):
        for metric in ("euclidean", "euclideanSquared"):
            print(f"ivf screen compact nprobe={nprobe} k={k} {metric} step={step}", flush=True)
            gd, gi = a.search(q, k, metric=metric)
            hd, hi = b.search(q, k, metric=metric)
            np.testing.assert_array_equal(gi, hi)
            np.testing.assert_array_equal(gd.view(np.uint32), hd.view(np.uint32))
            od, oi = O.ivf_search(q, x, ids, lists, c, nprobe, k,
                                  squared=metric != "euclidean")
            np.testing.assert_array_equal(gi, oi)
            np.testing.assert_array_equal(gd.view(np.uint32), od.view(np.uint32))
        # rows next to the queries, added after the plane and radii were made
        extra = (q[:20] + 0.05).astype(np.float32)
        eids = np.arange(len(x), len(x) + len(extra), dtype=np.int64) * 2 + 1
        a.insert(extra, eids)
        b.insert(extra, eids)
        x = np.concatenate([x, extra])
        ids = np.concatenate([ids, eids])
        lists = O.ivf_assign(x, c)
    assert "ivf_list_screen" in sctx.profile_stats()
    sctx.close()
    actx.close()


def test_ivf_build_one_call_matches_create_add(ctx):
    x, q, c = _mixture(11, 32, 6000, 40, 25)
    ids = np.arange(len(x), dtype=np.int64) * 5 + 1
    cfg = IVFConfiguration(dimensions=40, numberOfCentroids=32, numberOfProbes=6)
    for use_ids in (ids, None):
        print(f"ivf build ids={'given' if use_ids is not None else 'none'}", flush=True)
        built = IVFIndex.build(ctx, cfg, c, x, use_ids)
        ref = _index(ctx, c, x, use_ids, 6)
        np.testing.assert_array_equal(built.list_sizes(), ref.list_sizes())
        bd, bi = built.search(q, 12)
        rd, ri = ref.search(q, 12)
        np.testing.assert_array_equal(bi, ri)
        np.testing.assert_array_equal(bd, rd)
    empty = IVFIndex.build(ctx, cfg, c, x[:0])
    d, i = empty.search(q[:2], 3)
    assert (i == -1).all() and np.isinf(d).all()


def test_ivf_squared_metric_bit_exact(ctx):
    x, q, c = _mixture(12, 48, 12_000, 64, 60)
    ids = np.arange(len(x), dtype=np.int64)
    idx = _index(ctx, c, x, ids, 7)
    lists = O.ivf_assign(x, c)
    gd, gi = idx.search(q, 16, metric="euclideanSquared")
    od, oi = O.ivf_search(q, x, ids, lists, c, 7, 16, squared=True)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)


@pytest.mark.parametrize("metric", ["cosine", "dotProduct", "manhattan", "cosineNormalized"])
def test_ivf_rejects_non_euclidean_metric(ctx, metric):
    x, q, c = _mixture(13, 8, 500, 8, 4)
    idx = _index(ctx, c, x, None, 2)
    with pytest.raises(VSKError) as e:
        idx.search(q, 3, metric=metric)
    assert e.value.status == -8


def test_ivf_incremental_inserts_keep_order(ctx):
    x, q, c = _mixture(9, 20, 4000, 16, 30)
    idx = _index(ctx, c, None, nprobe=6)
    for part in np.array_split(np.arange(len(x)), 3):
        idx.insert(x[part], part.astype(np.int64))
    lists = O.ivf_assign(x, c)
    gd, gi = idx.search(q, 15)
    od, oi = O.ivf_search(q, x, np.arange(len(x), dtype=np.int64), lists, c, 6, 15)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)


def test_ivf_exact_strategy_equals_flat(ctx):
    x, q, c = _mixture(10, 24, 3000, 20, 25)
    idx = _index(ctx, c, x, nprobe=3)
    gd, gi = idx.search(q, 10, strategy="exact")
    fd, fi = O.search_flat(q, x, 10, O.L2)
    np.testing.assert_array_equal(gd, fd)
    for a, b in zip(gi, fi):
        assert set(a) == set(b)


def test_ivf_reference_kats(ctx):
    with open(os.path.join(GOLD, "reference_kats.json")) as f:
        k = json.load(f)["ivf_basic"]
    c = np.array(k["training"][:4], np.float32)
    idx = _index(ctx, c, np.array([k["inserted"]], np.float32), np.array([1], np.int64),
                 nprobe=k["nprobe"])
    d, i = idx.search(np.array([k["query"]], np.float32), 1)
    assert i[0, 0] == 1


def test_ivf_train_and_errors(ctx):
    x, q, c = _mixture(11, 8, 2000, 16, 5)
    cfg = KMeansClusteringConfiguration(maxIterations=5, initMethod="random", seed=0)
    idx = IVFIndex(ctx, IVFConfiguration(dimensions=16, numberOfCentroids=8, numberOfProbes=2,
                                         clusteringConfig=cfg))
    with pytest.raises(VSKError) as e:
        idx.search(q, 3)
    assert e.value.kind == "notTrained"
    idx.train(x)
    idx.insert(x)
    d, i = idx.search(q, 5, strategy="exact")
    fd, fi = O.search_flat(q, x, 5, O.L2)
    np.testing.assert_array_equal(d, fd)
    # empty lists and k > candidates pad with (inf, -1)
    empty = _index(ctx, c, None, nprobe=2)
    d, i = empty.search(q, 4)
    assert (i == -1).all() and np.isinf(d).all()


def test_config3_full_size(ctx):
    """1M x 128 from a 4,096-Gaussian mixture, nlist 4096,
    nprobe 32, 10,000 queries, k=10.  Assignment checked bit-exact on a row
    sample, search bit-exact on all 10,000 queries, recall@10 vs exact search
    equal to the oracle's on the first 1,000."""
    import torch

    n, d, ncent, nq, nprobe, k = 1_000_000, 128, 4096, 10_000, 32, 10
    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    cent = 2.0 * torch.randn(ncent, d, generator=g, device="cuda")
    g.manual_seed(5)
    a = torch.randint(0, ncent, (n,), generator=g, device="cuda")
    qa = torch.randint(0, ncent, (nq,), generator=g, device="cuda")
    g.manual_seed(1)
    x = cent[a] + 0.5 * torch.randn(n, d, generator=g, device="cuda")
    g.manual_seed(2)
    q = cent[qa] + 0.5 * torch.randn(nq, d, generator=g, device="cuda")
    g.manual_seed(4)
    c = cent + 0.1 * torch.randn(ncent, d, generator=g, device="cuda")
    xh, qh, ch = x.cpu().numpy(), q.cpu().numpy(), c.cpu().numpy()
    print("config3 ivf 1Mx128 nlist4096 nprobe32 q10000 k10", flush=True)
    idx = _index(ctx, ch, x, nprobe=nprobe)
    lists = idx.assign(x).cpu().numpy()
    sample = np.random.default_rng(0).choice(n, 20_000, replace=False)
    np.testing.assert_array_equal(lists[sample], O.ivf_assign(xh[sample], ch))
    gd, gi = idx.search(q, k)
    gd, gi = gd.cpu().numpy(), gi.cpu().numpy()
    assert_sorted_unique(gd, gi)
    od, oi = O.ivf_search(qh, xh, np.arange(n, dtype=np.int64), lists, ch, nprobe, k)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd.view(np.uint32), od.view(np.uint32))
    sub = 1000
    td, ti = O.search_flat(qh[:sub], xh, k, O.L2)
    assert recall(gi[:sub], ti) == recall(oi[:sub], ti)
    print(f"config3 recall@10 on {sub} queries: {recall(gi[:sub], ti):.4f}", flush=True)

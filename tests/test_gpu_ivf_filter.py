"""IVF search with a row filter and after row removal, against the oracle
over the surviving rows.

The reference filters the probed lists' candidates and then ranks them
(Indexes/IVFIndex.swift:154-176; applyFilter :161-165), and delete removes
the row from its list (:210-220).  The probes do not depend on the rows, so
the oracle's answer is the IVF search over the surviving rows in their list
order (their ids kept): bit-exact distances and ids at any selectivity."""
import os

import numpy as np
import pytest

from oracle import oracle as O
from vectorstorekit_amd import (Context, IVFConfiguration, IVFIndex, ScalarQuantizer,
                                VSKError)

pytestmark = pytest.mark.gpu


def _mixture(seed, ncent, n, d, nq):
    rng = np.random.default_rng(seed)
    cent = (2.0 * rng.standard_normal((ncent, d))).astype(np.float32)
    a = rng.integers(0, ncent, n)
    x = (cent[a] + 0.5 * rng.standard_normal((n, d))).astype(np.float32)
    qa = rng.integers(0, ncent, nq)
    q = (cent[qa] + 0.5 * rng.standard_normal((nq, d))).astype(np.float32)
    c = (cent + 0.1 * rng.standard_normal(cent.shape)).astype(np.float32)
    return x, q, c


def _index(ctx, c, x, nprobe):
    idx = IVFIndex(ctx, IVFConfiguration(dimensions=c.shape[1], numberOfCentroids=c.shape[0],
                                         numberOfProbes=nprobe))
    idx.set_centroids(c)
    if x is not None:
        idx.insert(x)  # ids 0, 1, 2, ... (the running count)
    return idx


def _screen_ctx():
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


def _oracle(q, x, keep, lists, c, nprobe, k, sq=False):
    sub = np.flatnonzero(keep)
    return O.ivf_search(q, x[sub], sub.astype(np.int64), lists[sub], c, nprobe, k, squared=sq)


def _same(g, o):
    np.testing.assert_array_equal(np.asarray(g[1]), o[1])
    np.testing.assert_array_equal(np.asarray(g[0]).view(np.uint32), o[0].view(np.uint32))


# (nlist, n, d, nq, nprobe, k, fraction kept, screen, metric)
SHAPES = [(64, 20_000, 128, 200, 8, 10, 0.005, False, "euclidean"),
          (37, 5000, 33, 60, 5, 7, 0.3, False, "euclideanSquared"),
          (64, 20_000, 128, 200, 8, 10, 0.005, True, "euclidean"),
          (40, 12_000, 160, 90, 40, 100, 0.02, True, "euclidean"),
          (24, 9000, 256, 70, 6, 64, 0.5, True, "euclideanSquared"),
          (32, 15_000, 64, 30, 12, 300, 0.5, True, "euclidean")]


@pytest.mark.parametrize("shape", SHAPES)
def test_ivf_filtered_bit_exact(ctx, shape):
    """Filters that keep 0.5 % to 50 % of the rows, on the exact list scan
    and on the bf16 screen (k up to 64 through the fused tail, 100, and 300
    through separate margin, rescore and redo launches); filters given as a
    boolean mask and as allowed ids; a filter that keeps nothing."""
    nlist, n, d, nq, nprobe, k, frac, screen, metric = shape
    print(f"ivf filter nlist={nlist} n={n} d={d} nq={nq} nprobe={nprobe} k={k} "
          f"keep={frac} screen={screen} {metric}", flush=True)
    sq = metric == "euclideanSquared"
    x, q, c = _mixture(nlist * 7 + n, nlist, n, d, nq)
    uctx = _screen_ctx() if screen else ctx
    idx = _index(uctx, c, x, nprobe)
    lists = O.ivf_assign(x, c)
    rng = np.random.default_rng(n + k)
    keep = rng.random(n) < frac
    _same(idx.search(q, k, metric=metric, allow=keep),
          _oracle(q, x, keep, lists, c, nprobe, k, sq))
    if screen:
        assert "ivf_list_screen" in uctx.profile_stats(), "the screen did not run"
        assert "ivf_mask_words" in uctx.profile_stats(), "the filter did not run"
    # as allowed ids, with the bitmap ending before the last rows (the rows
    # it does not reach are excluded)
    ids = np.flatnonzero(keep[: n - 97])
    keep2 = np.zeros(n, np.bool_)
    keep2[ids] = True
    _same(idx.search(q, k, metric=metric, allow=ids, allow_bits=n - 97),
          _oracle(q, x, keep2, lists, c, nprobe, k, sq))
    # nothing passes
    gd, gi = idx.search(q[:3], k, metric=metric, allow=np.zeros(n, np.bool_))
    assert (np.asarray(gi) == -1).all() and np.isinf(np.asarray(gd)).all()
    if screen:
        uctx.close()


@pytest.mark.parametrize("k", [10, 300])
def test_ivf_filtered_margin_overflow(k):
    """Through the screen, a block of identical rows next to the first
    query, more of them passing the filter than the margin's slots hold
    (1,024; 4k above k = 256): that query's whole candidate set is rescored
    (the tail's fallback, or the separate redo launch), and the rows the
    filter rejects must stay out of it."""
    nlist, n, d, nq, nprobe = 32, 8000, 64, 20, 6
    x, q, c = _mixture(4242 + k, nlist, n, d, nq)
    rng = np.random.default_rng(k)
    ndup = max(2400, 6 * k + 300)
    dup = np.repeat(q[:1] + 0.01 * rng.standard_normal((1, d)).astype(np.float32), ndup, 0)
    x2 = np.concatenate([x, dup]).astype(np.float32)
    sctx = _screen_ctx()
    idx = _index(sctx, c, x2, nprobe)
    lists = O.ivf_assign(x2, c)
    keep = rng.random(len(x2)) < 0.7
    keep[n:] = np.arange(ndup) % 3 != 0  # two thirds of the copies pass
    fallback = "ivf_screen_tail" if k <= 256 else "ivf_screen_redo"
    before = sctx.profile_stats().get(fallback, (0, 0.0, 0.0))[2]
    _same(idx.search(q, k, allow=keep), _oracle(q, x2, keep, lists, c, nprobe, k))
    assert sctx.profile_stats()[fallback][2] > before, "no query overflowed"
    sctx.close()


def test_ivf_remove_bit_exact(ctx):
    """vsk_ivf_remove: the removed rows leave their lists, the others keep
    their list order, so searches (exact scan and screen), list sizes and
    the lists' ids equal the index of the surviving rows; SQ8 codes stay
    valid; later inserts continue the ids; removing unknown ids removes
    nothing; removing every row leaves an empty index."""
    nlist, n, d, nq, nprobe, k = 48, 20_000, 96, 80, 8, 20
    x, q, c = _mixture(99, nlist, n, d, nq)
    idx = _index(ctx, c, x, nprobe)
    sq = ScalarQuantizer(ctx, per_dim=True)
    sq.train(x)
    idx.encodeSQ8(sq)
    lists = O.ivf_assign(x, c)
    near = O.search_flat(q[:1], x, 300, O.L2)[1][0]
    gone = np.unique(np.concatenate([near, np.random.default_rng(1).choice(n, 1000)]))
    assert idx.remove(np.concatenate([gone, gone[:5]])) == gone.size  # duplicates once
    keep = np.ones(n, np.bool_)
    keep[gone] = False
    _same(idx.search(q, k), _oracle(q, x, keep, lists, c, nprobe, k))
    np.testing.assert_array_equal(idx.list_sizes(), np.bincount(lists[keep], minlength=nlist))
    lids, off = idx.listIds()
    sub = np.flatnonzero(keep)
    order = np.argsort(lists[sub], kind="stable")
    np.testing.assert_array_equal(lids, sub[order])
    np.testing.assert_array_equal(off[1:], np.cumsum(np.bincount(lists[sub], minlength=nlist)))
    # SQ8 codes of the kept rows
    score, ids = idx.searchSQ8(q, k)
    codes = O.sq8_encode(x, sq.scale, sq.offset)
    qc = O.sq8_encode(q, sq.scale, sq.offset)
    es, ei = O.ivf_sq8_search(q, qc, codes[sub], sub, lists[sub], c, nprobe, k)
    np.testing.assert_array_equal(score, es)
    np.testing.assert_array_equal(ids, ei)
    # the screen over the rows left (its plane is made again)
    sctx = _screen_ctx()
    sidx = _index(sctx, c, x, nprobe)
    assert sidx.remove(gone) == gone.size
    _same(sidx.search(q, k), _oracle(q, x, keep, lists, c, nprobe, k))
    assert "ivf_list_screen" in sctx.profile_stats()
    sidx.free()
    sctx.close()
    # ids continue after a removal; unknown ids remove nothing
    extra = x[:50] + 0.25
    idx.insert(extra)
    x2 = np.concatenate([x, extra])
    keep2 = np.concatenate([keep, np.ones(50, np.bool_)])
    _same(idx.search(q, k), _oracle(q, x2, keep2, O.ivf_assign(x2, c), c, nprobe, k))
    assert idx.remove([n + 10**6, -5]) == 0
    with pytest.raises(VSKError):  # rows added after the codes were made
        idx.searchSQ8(q, k)
    # everything
    assert idx.remove(np.arange(n + 50)) == keep2.sum()
    gd, gi = idx.search(q[:2], k)
    assert (np.asarray(gi) == -1).all() and np.isinf(np.asarray(gd)).all()
    assert idx.list_sizes().sum() == 0


def test_config3_filter_and_delete(ctx):
    """BASELINE config 3's index (1M x 128, nlist 4096, nprobe 32): a filter
    that keeps 0.5 % of the rows, and a query batch whose 2,000 nearest rows
    each are removed, at k = 10 and k = 100, on the exact list scan (200
    queries) and through the screen (2,000 queries, past its size
    threshold), bit-exact against the oracle over the surviving rows."""
    import torch

    n, d, ncent, nprobe = 1_000_000, 128, 4096, 32
    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    cent = 2.0 * torch.randn(ncent, d, generator=g, device="cuda")
    g.manual_seed(5)
    a = torch.randint(0, ncent, (n,), generator=g, device="cuda")
    qa = torch.randint(0, ncent, (2000,), generator=g, device="cuda")
    g.manual_seed(1)
    x = cent[a] + 0.5 * torch.randn(n, d, generator=g, device="cuda")
    g.manual_seed(2)
    q = cent[qa] + 0.5 * torch.randn(2000, d, generator=g, device="cuda")
    g.manual_seed(4)
    c = cent + 0.1 * torch.randn(ncent, d, generator=g, device="cuda")
    xh, qh, ch = x.cpu().numpy(), q.cpu().numpy(), c.cpu().numpy()
    idx = _index(ctx, ch, x, nprobe)
    lists = idx.assign(x).cpu().numpy()
    keep = np.random.default_rng(11).random(n) < 0.005
    for k in (10, 100):
        for nq in (200, 2000):
            print(f"config3 filter keep=0.005 k={k} nq={nq}", flush=True)
            _same([t.cpu().numpy() for t in idx.search(q[:nq], k, allow=keep)],
                  _oracle(qh[:nq], xh, keep, lists, ch, nprobe, k))
    # the 2,000 nearest rows of each of the first 4 queries leave the index
    near = O.search_flat(qh[:4], xh, 2000, O.L2)[1]
    gone = np.unique(near)
    print(f"config3 remove {gone.size} rows", flush=True)
    assert idx.remove(gone) == gone.size
    alive = np.ones(n, np.bool_)
    alive[gone] = False
    for k in (10, 100):
        for nq in (200, 2000):
            print(f"config3 after delete k={k} nq={nq}", flush=True)
            _same([t.cpu().numpy() for t in idx.search(q[:nq], k)],
                  _oracle(qh[:nq], xh, alive, lists, ch, nprobe, k))
    # the first queries' results hold none of their removed neighbours
    gd, gi = idx.search(qh[:4], 100)
    for i in range(4):
        assert not set(gi[i].tolist()) & set(near[i].tolist())


def test_exact_strategy_ties_follow_probe_order(ctx):
    """.exact over more lists than a selection holds (1,100 > 1,024): the
    reference concatenates the lists in findNearestCentroids' order (by
    distance, then centroid index) and stable-sorts, so of two rows at
    exactly the same distance the one in the nearer list comes first even
    when its centroid index is higher.  Rows +-delta*e0 around the query
    (distance delta both) sit in list 5 (far) and list 900 (near)."""
    d, nlist = 8, 1100
    rng = np.random.default_rng(17)
    c = (100.0 + 10.0 * rng.standard_normal((nlist, d))).astype(np.float32)
    delta = np.float32(0.25)
    c[5] = 0
    c[5, 0] = 2 * delta          # nearest to +delta e0; 2 delta from the query
    c[900] = 0
    c[900, 0] = -1.5 * delta     # nearest to -delta e0; 1.5 delta from the query
    x = (100.0 + 10.0 * rng.standard_normal((3000, d))).astype(np.float32)
    a = np.zeros(d, np.float32)
    a[0] = delta
    x[100], x[2000] = a, -a       # row 100 in list 5, row 2000 in list 900
    q = np.zeros((1, d), np.float32)
    idx = _index(ctx, c, x, 8)
    lists = O.ivf_assign(x, c)
    assert lists[100] == 5 and lists[2000] == 900
    gd, gi = idx.search(q, 2, strategy="exact")
    od, oi = O.ivf_search(q, x, np.arange(len(x)), lists, c, nlist, 2)
    assert list(oi[0]) == [2000, 100]
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)
    # and with more queries and rows, every result
    q2 = (100.0 + 10.0 * rng.standard_normal((40, d))).astype(np.float32)
    x2 = np.concatenate([x, x[:500]])  # exact duplicates in the same lists
    idx2 = _index(ctx, c, x2, 8)
    gd, gi = idx2.search(q2, 20, strategy="exact")
    od, oi = O.ivf_search(q2, x2, np.arange(len(x2)), O.ivf_assign(x2, c), c, nlist, 20)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)

"""Shared parity checks for GPU results against the CPU oracle."""
import numpy as np


def assert_topk_match(gd, gi, od, oi, dist_fn, rtol=1e-4, atol=1e-4):
    """GPU top-k (gd, gi) against the oracle's (od, oi), the float-path bar:
    distances at every rank within rtol relative (+atol for values near 0),
    and id sets identical except for ids whose oracle distance ties the
    k-th distance within that tolerance.  dist_fn(query_index, ids) returns
    the oracle's distances of those ids."""
    gd, gi, od, oi = map(np.asarray, (gd, gi, od, oi))
    assert gd.shape == od.shape and gi.shape == oi.shape
    finite = np.isfinite(od)
    np.testing.assert_array_equal(np.isfinite(gd), finite)
    np.testing.assert_allclose(gd[finite], od[finite], rtol=rtol, atol=atol)
    assert (gi[~finite] == -1).all()
    for q in range(gi.shape[0]):
        a = set(gi[q][gi[q] >= 0].tolist())
        b = set(oi[q][oi[q] >= 0].tolist())
        if a == b:
            continue
        kth = od[q][finite[q]][-1]
        tol = rtol * abs(kth) + atol
        extra = np.array(sorted(a - b), np.int64)
        missing = np.array(sorted(b - a), np.int64)
        assert len(extra) == len(missing), (q, extra, missing)
        de = dist_fn(q, extra)
        dm = dist_fn(q, missing)
        assert np.all(np.abs(de - kth) <= tol), (q, extra, de, kth)
        assert np.all(np.abs(dm - kth) <= tol), (q, missing, dm, kth)


def assert_sorted_unique(dist, ids):
    dist, ids = np.asarray(dist), np.asarray(ids)
    assert (np.diff(dist, axis=1) >= 0).all() or np.isnan(dist).any()
    for row in ids:
        v = row[row >= 0]
        assert len(np.unique(v)) == len(v)


def recall(found, truth):
    found, truth = np.asarray(found), np.asarray(truth)
    hit = 0
    for f, t in zip(found, truth):
        hit += len(set(f.tolist()) & set(t.tolist()))
    return hit / truth.size

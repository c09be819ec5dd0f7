"""Searches are queued whole and wait for the GPU once: the progressive
top-k no longer reads an overflow count back after each filtered chunk, and
the flat screen no longer waits for its bound check (both come back with the
call's final synchronisation).  vsk_last_sync_count reports the host waits of
the last call; each search here runs once to build its planes and scratch,
then again, and the second call must wait exactly once, with results still
bit-exact against the oracle.  A forced overflow takes the checked path
(more waits) and stays exact."""
import numpy as np
import pytest

from oracle import oracle as O
from vectorstorekit_amd import (BinaryDatabase, BinaryQuantizer, IVFConfiguration, IVFIndex,
                                ProductQuantizer, SQ8Database, VectorDatabase)
from vectorstorekit_amd._lib import (METRIC_COSINE, METRIC_COSINE_NORMALIZED, METRIC_L1,
                                     METRIC_L2SQ)

pytestmark = pytest.mark.gpu


def _twice(ctx, fn):
    fn()
    out = fn()
    return out, ctx.last_sync_count()


def test_flat_screen_one_wait(ctx):
    """Normalised cosine through the screen (a dense first chunk and several
    filtered ones), k = 100."""
    rng = np.random.default_rng(1)
    n, nq, d, k = 300_000, 600, 128, 100
    x = rng.standard_normal((n, d)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    q = rng.standard_normal((nq, d)).astype(np.float32)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    print(f"one-sync flat screen n={n} nq={nq} d={d} k={k}", flush=True)
    db = VectorDatabase(ctx, x)
    (gd, gi), waits = _twice(ctx, lambda: db.search(q, k, METRIC_COSINE_NORMALIZED))
    od, oi = O.search_flat(q, x, k, METRIC_COSINE_NORMALIZED)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)
    assert waits == 1, f"{waits} host waits"
    # the epsilon cosine: its relative bound is made once per database (one
    # more wait in the first call), then one wait a call
    xs = x * rng.uniform(0.5, 4.0, (n, 1)).astype(np.float32)
    db2 = VectorDatabase(ctx, xs)
    (gd, gi), waits = _twice(ctx, lambda: db2.search(q, k, METRIC_COSINE))
    od, oi = O.search_flat(q, xs, k, METRIC_COSINE)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)
    assert waits == 1, f"{waits} host waits (cosine)"


def test_sq8_one_wait(ctx):
    rng = np.random.default_rng(2)
    n, nq, d, k = 2_000_000, 200, 128, 100
    codes = rng.integers(-128, 128, (n, d), dtype=np.int8)
    qc = rng.integers(-128, 128, (nq, d), dtype=np.int8)
    print(f"one-sync sq8 n={n} nq={nq} k={k}", flush=True)
    db = SQ8Database(ctx, codes)
    (gs, gi), waits = _twice(ctx, lambda: db.search(qc, k))
    os_, oi = O.sq8_search(qc, codes, k)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gs, os_)
    assert waits == 1, f"{waits} host waits"


def test_pq_and_binary_one_wait(ctx):
    rng = np.random.default_rng(3)
    n, nq, M, dsub, k = 1_000_000, 300, 16, 8, 100
    books = rng.standard_normal((M, 256, dsub)).astype(np.float32)
    codes = rng.integers(0, 256, (n, M), dtype=np.uint8)
    q = rng.standard_normal((nq, M * dsub)).astype(np.float32)
    print(f"one-sync pq n={n} nq={nq} k={k}", flush=True)
    pq = ProductQuantizer.upload(ctx, books, codes)
    (gd, gi), waits = _twice(ctx, lambda: pq.search(q, k, k_adc=k))
    od, oi = O.pq_search(q, books, codes, k, k)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)
    assert waits == 1, f"pq: {waits} host waits"
    x = rng.standard_normal((n, 128)).astype(np.float32)
    bq = BinaryQuantizer(ctx)
    bdb = BinaryDatabase(ctx, bq.quantizeBatch(x), d=128)
    qb = bq.quantizeBatch(q[:, :128].copy())
    (hd, hi), waits = _twice(ctx, lambda: bdb.search(qb, k))
    assert waits == 1, f"binary: {waits} host waits"


def test_ivf_one_wait(ctx):
    rng = np.random.default_rng(4)
    nlist, n, d, nq, nprobe, k = 256, 200_000, 64, 2000, 16, 10
    cent = (2.0 * rng.standard_normal((nlist, d))).astype(np.float32)
    x = (cent[rng.integers(0, nlist, n)] + 0.5 * rng.standard_normal((n, d))).astype(np.float32)
    q = (cent[rng.integers(0, nlist, nq)] + 0.5 * rng.standard_normal((nq, d))).astype(np.float32)
    idx = IVFIndex(ctx, IVFConfiguration(dimensions=d, numberOfCentroids=nlist,
                                         numberOfProbes=nprobe))
    idx.set_centroids(cent)
    idx.insert(x)
    print(f"one-sync ivf n={n} nq={nq} k={k}", flush=True)
    (gd, gi), waits = _twice(ctx, lambda: idx.search(q, k))
    od, oi = O.ivf_search(q, x, np.arange(n), O.ivf_assign(x, cent), cent, nprobe, k)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)
    assert waits == 1, f"{waits} host waits"


def test_overflow_takes_checked_path(ctx):
    """Rows strictly closer with growing id: every filtered chunk overflows,
    the call notices at its end and runs again with a check per chunk."""
    n = 120_000
    x = np.zeros((n, 4), np.float32)
    x[:, 0] = np.arange(n, dtype=np.float32) / n
    q = np.array([[2.0, 0, 0, 0], [-1.0, 0, 0, 0]], np.float32)
    db = VectorDatabase(ctx, x)
    (gd, gi), waits = _twice(ctx, lambda: db.search(q, 10, METRIC_L1))
    od, oi = O.search_flat(q, x, 10, METRIC_L1)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)
    assert waits > 2, f"{waits} host waits: the overflow was not seen"

"""VSK_MAX_TILE_BYTES: a context whose working buffers per query batch are
capped splits every search into many query batches (as the reference's
MetalDistanceCompute chunks queries under its buffer limit,
Acceleration/Metal/MetalDistanceCompute.swift:371-380,450-473).  The answers
must not depend on the chunking: bit-identical to the default context's for
the flat screen and exact scan, SQ8, PQ (screen and LUT), binary and IVF
(screen and exact scan), and equal to the oracle."""
import os

import numpy as np
import pytest

from oracle import oracle as O
from vectorstorekit_amd import (BinaryDatabase, BinaryQuantizer, Context, IVFConfiguration,
                                IVFIndex, ProductQuantizer, SQ8Database, VectorDatabase)
from vectorstorekit_amd._lib import METRIC_COSINE_NORMALIZED, METRIC_L1, METRIC_L2

pytestmark = pytest.mark.gpu


def _ctx(**env):
    old = {k: os.environ.get(k) for k in env}
    os.environ.update({k: str(v) for k, v in env.items()})
    try:
        return Context(0)
    finally:
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v


@pytest.mark.parametrize("screen", [False, True])
def test_chunk_invariance(ctx, screen):
    rng = np.random.default_rng(31 + screen)
    kern = {"VSK_FLAT_KERNEL": "screen"} if screen else {}
    small = _ctx(VSK_MAX_TILE_BYTES=1 << 16, **kern)  # a few queries a batch
    base = _ctx(**kern) if screen else ctx
    print(f"tile-bytes chunking screen={screen}", flush=True)
    # flat: normalised cosine (screen or exact VALU scan) and L1
    x = rng.standard_normal((30_000, 96)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    q = rng.standard_normal((70, 96)).astype(np.float32)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    for metric in (METRIC_COSINE_NORMALIZED, METRIC_L1):
        a = VectorDatabase(base, x).search(q, 50, metric)
        b = VectorDatabase(small, x).search(q, 50, metric)
        np.testing.assert_array_equal(a[1], b[1])
        np.testing.assert_array_equal(a[0], b[0])
        od, oi = O.search_flat(q, x, 50, metric)
        np.testing.assert_array_equal(b[1], oi)
        np.testing.assert_array_equal(b[0], od)
    # SQ8
    codes = rng.integers(-128, 128, (50_000, 64)).astype(np.int8)
    qc = rng.integers(-128, 128, (40, 64)).astype(np.int8)
    a = SQ8Database(base, codes).search(qc, 30)
    b = SQ8Database(small, codes).search(qc, 30)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])
    # PQ with an L1 re-rank
    books = rng.standard_normal((8, 256, 4)).astype(np.float32)
    pcodes = rng.integers(0, 256, (40_000, 8), dtype=np.uint8)
    pq_a = ProductQuantizer.upload(base, books, pcodes)
    pq_b = ProductQuantizer.upload(small, books, pcodes)
    xq = rng.standard_normal((40_000, 32)).astype(np.float32)
    qq = rng.standard_normal((30, 32)).astype(np.float32)
    a = pq_a.search(qq, 20, k_adc=200, rerank_metric="manhattan",
                    rerank_db=VectorDatabase(base, xq))
    b = pq_b.search(qq, 20, k_adc=200, rerank_metric="manhattan",
                    rerank_db=VectorDatabase(small, xq))
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])
    # binary
    bq = BinaryQuantizer(base)
    bc = bq.quantizeBatch(rng.standard_normal((20_000, 128)).astype(np.float32))
    qb = bq.quantizeBatch(rng.standard_normal((25, 128)).astype(np.float32))
    a = BinaryDatabase(base, bc, 128).search(qb, 40)
    b = BinaryDatabase(small, bc, 128).search(qb, 40)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])
    # IVF
    cent = (2.0 * rng.standard_normal((64, 48))).astype(np.float32)
    xi = (cent[rng.integers(0, 64, 30_000)] + 0.5 * rng.standard_normal((30_000, 48))).astype(
        np.float32)
    qi = (cent[rng.integers(0, 64, 300)] + 0.5 * rng.standard_normal((300, 48))).astype(
        np.float32)
    res = []
    for c in (base, small):
        idx = IVFIndex(c, IVFConfiguration(dimensions=48, numberOfCentroids=64,
                                           numberOfProbes=6))
        idx.set_centroids(cent)
        idx.insert(xi)
        res.append(idx.search(qi, 15))
        idx.free()
    np.testing.assert_array_equal(res[0][1], res[1][1])
    np.testing.assert_array_equal(res[0][0], res[1][0])
    od, oi = O.ivf_search(qi, xi, np.arange(len(xi)), O.ivf_assign(xi, cent), cent, 6, 15)
    np.testing.assert_array_equal(res[1][1], oi)
    np.testing.assert_array_equal(res[1][0], od)
    small.close()
    if screen:
        base.close()


def test_configure_round_trip_and_effect():
    """vsk_configure sets what the environment sets at creation: the
    kernel choice (exact: no screen ran), profiling and the tile budget."""
    from vectorstorekit_amd import HIPAccelerationConfiguration

    cfg = HIPAccelerationConfiguration(kernel="exact", enableProfiling=True,
                                       maxTileBytes=1 << 20)
    c = Context(0, cfg)
    got = c.configuration()
    assert (got.kernel, got.enableProfiling, got.maxTileBytes) == ("exact", True, 1 << 20)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((200_000, 64)).astype(np.float32)
    q = rng.standard_normal((300, 64)).astype(np.float32)
    gd, gi = VectorDatabase(c, x).search(q, 20, "euclideanSquared")
    assert "flat_screen_filter" not in c.profile_stats()
    od, oi = O.search_flat(q, x, 20, O.L2SQ)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)
    c.configure(HIPAccelerationConfiguration(kernel="screen", enableProfiling=True))
    c.profile_reset()
    gd2, gi2 = VectorDatabase(c, x).search(q, 20, "euclideanSquared")
    assert "flat_screen_filter" in c.profile_stats()
    np.testing.assert_array_equal(gi2, oi)
    np.testing.assert_array_equal(gd2, od)
    c.close()

"""Double-run determinism: every main kernel path run twice on the same
inputs returns identical bytes (a race on LDS or on the candidate lists
would show as run-to-run differences).  The exact paths are also checked
against the oracle elsewhere; this covers the tolerance paths (bf16x3
cosine, the fp32 MFMA kernel) and the candidate order of every path, with
the screen forced at small sizes and every search repeated on a fresh
context as well."""
import os

import numpy as np
import pytest

from oracle import oracle as O
from vectorstorekit_amd import (Context, IVFConfiguration, IVFIndex, ProductQuantizer,
                                SQ8Database, ScalarQuantizer, VectorDatabase)

pytestmark = pytest.mark.gpu


def _context(kernel):
    old = os.environ.get("VSK_FLAT_KERNEL")
    if kernel is None:
        os.environ.pop("VSK_FLAT_KERNEL", None)
    else:
        os.environ["VSK_FLAT_KERNEL"] = kernel
    try:
        return Context(0)
    finally:
        if old is None:
            os.environ.pop("VSK_FLAT_KERNEL", None)
        else:
            os.environ["VSK_FLAT_KERNEL"] = old


def _twice(make, run):
    """run(obj) on one context twice, then on a fresh context: all equal."""
    outs = []
    for fresh in (False, False, True):
        if fresh or not outs:
            obj, ctx = make()
        outs.append([np.array(a, copy=True) for a in run(obj)])
    for o in outs[1:]:
        for a, b in zip(outs[0], o):
            assert a.dtype == b.dtype and a.shape == b.shape
            assert a.tobytes() == b.tobytes()


@pytest.mark.parametrize("kernel,metric", [("screen", "cosineNormalized"),
                                           ("screen", "euclideanSquared"),
                                           ("bf16x3", "cosine"), ("fp32", "euclidean"),
                                           (None, "manhattan")])
def test_flat_twice(kernel, metric):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((12_000, 96)).astype(np.float32)
    q = rng.standard_normal((70, 96)).astype(np.float32)
    if metric == "cosineNormalized":
        x /= np.linalg.norm(x, axis=1, keepdims=True)
        q /= np.linalg.norm(q, axis=1, keepdims=True)

    def make():
        ctx = _context(kernel)
        return VectorDatabase(ctx, x), ctx

    _twice(make, lambda db: db.search(q, 40, metric))


def test_sq8_twice():
    rng = np.random.default_rng(12)
    x = rng.standard_normal((60_000, 128)).astype(np.float32)
    q = rng.standard_normal((200, 128)).astype(np.float32)
    s, o = O.sq8_train(x, per_dim=True)
    codes, qc = O.sq8_encode(x, s, o), O.sq8_encode(q, s, o)

    def make():
        ctx = Context(0)
        return SQ8Database(ctx, codes), ctx

    _twice(make, lambda db: db.search(qc, 50))


def test_pq_screen_twice():
    rng = np.random.default_rng(13)
    n, d, M = 40_000, 64, 8
    x = rng.standard_normal((n, d)).astype(np.float32)
    q = rng.standard_normal((50, d)).astype(np.float32)
    cb = rng.standard_normal((M, 256, d // M)).astype(np.float32)
    codes = O.pq_encode(x, cb)

    def make():
        ctx = _context("screen")
        pq = ProductQuantizer(ctx, cb)
        pq.add(codes)
        return pq, ctx

    _twice(make, lambda pq: pq.search(q, 20, k_adc=300))


def test_ivf_twice():
    rng = np.random.default_rng(14)
    d, nlist = 64, 50
    cent = (2.0 * rng.standard_normal((nlist, d))).astype(np.float32)
    x = (cent[rng.integers(0, nlist, 30_000)]
         + 0.5 * rng.standard_normal((30_000, d))).astype(np.float32)
    q = (cent[rng.integers(0, nlist, 300)] + 0.5 * rng.standard_normal((300, d))).astype(np.float32)

    def make():
        ctx = _context("screen")
        idx = IVFIndex(ctx, IVFConfiguration(dimensions=d, numberOfCentroids=nlist,
                                             numberOfProbes=6))
        idx.set_centroids(cent)
        idx.insert(x)
        return idx, ctx

    _twice(make, lambda idx: idx.search(q, 10))

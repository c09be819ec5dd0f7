"""Pins the CPU oracle's distance and top-k functions.

Known answers are the reference's own closed-form tests (paths relative to
Tests/VectorStoreKitTests/ of gifton/VectorStoreKit); the rest is checked
against float64 numpy and brute force, which a dropped term, a wrong sign or
a transposed operand in the oracle would fail.
"""
import json
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def kats():
    with open(os.path.join(GOLD, "reference_kats.json")) as f:
        return json.load(f)


def _const(v, d):
    return np.full(d, v, np.float32)


def test_vector512_kats():
    # Vector512Tests.swift:61-67, 69-78, 144-159
    k = kats()["vector512"]
    one, two, three, zero = (_const(v, 512) for v in (1, 2, 3, 0))
    assert O.distance(one, two, O.DOT) == pytest.approx(-k["dot_1_2"], abs=1e-3)
    assert O.distance(one, three, O.L2SQ) == pytest.approx(k["l2sq_1_3"], abs=1e-3)
    assert O.distance(zero, one, O.L2) == pytest.approx(k["l2_0_1"], abs=1e-3)
    assert O.distance(zero, one, O.L1) == pytest.approx(k["l1_0_1"], abs=1e-3)


def test_cosine_kats():
    # Vector512Tests.swift:80-102: parallel unit vectors -> similarity 1,
    # orthogonal -> 0; the distance form is 1 - similarity.
    k = kats()["vector512"]
    v = _const(1, 512) / np.sqrt(512)
    assert 1 - O.distance(v, v, O.COSINE_NORMALIZED) == pytest.approx(k["cos_parallel"], abs=1e-3)
    assert 1 - O.distance(v, v, O.COSINE) == pytest.approx(k["cos_parallel"], abs=1e-3)
    e0 = np.zeros(512, np.float32)
    e0[0] = 1
    e1 = np.zeros(512, np.float32)
    e1[1] = 1
    assert 1 - O.distance(e0, e1, O.COSINE) == pytest.approx(k["cos_orthogonal"], abs=1e-3)


def test_batch_constant_kat():
    # Vector512Tests.swift:174-204 and MetalDistance512Tests.swift:50-66:
    # query 0 vs candidate rows filled with i -> sqrt(512 i^2)
    k = kats()["batch_constant"]
    x = np.stack([_const(i, 512) for i in range(100)])
    d = O.distances(_const(0, 512)[None], x, O.L2)[0]
    np.testing.assert_allclose(d[:2], k["first_two"], atol=1e-3)
    np.testing.assert_allclose(d, np.sqrt(512.0) * np.arange(100), rtol=1e-6)


def test_distance_matrix_kats():
    # MetalDistanceMatrixTests.swift:27-55 (symmetric, zero diagonal) and
    # :76-111 (0 vs 1: L2 sqrt(512), L1 512, cosine of parallel 0)
    k = kats()["distance_matrix"]
    rng = np.random.default_rng(0)
    v = rng.standard_normal((20, 64)).astype(np.float32)
    for m in (O.L2, O.L1):
        D = O.distances(v, v, m)
        np.testing.assert_allclose(D, D.T, rtol=1e-6, atol=1e-6)
        np.testing.assert_allclose(np.diag(D), 0, atol=0)
    z, o = _const(0, 512), _const(1, 512)
    assert O.distance(z, o, O.L2) == pytest.approx(k["l2_0_1"], abs=1e-3)
    assert O.distance(z, o, O.L1) == pytest.approx(k["l1_0_1"], abs=1e-3)
    assert O.distance(o, o * 3, O.COSINE) == pytest.approx(k["cos_parallel_distance"], abs=1e-3)


@pytest.mark.parametrize("metric", [O.L2SQ, O.L2, O.COSINE, O.COSINE_NORMALIZED, O.DOT, O.L1])
def test_distances_vs_float64(metric):
    rng = np.random.default_rng(1 + metric)
    q = rng.standard_normal((7, 37)).astype(np.float32)
    x = rng.standard_normal((53, 37)).astype(np.float32)
    if metric == O.COSINE_NORMALIZED:
        q /= np.linalg.norm(q, axis=1, keepdims=True)
        x /= np.linalg.norm(x, axis=1, keepdims=True)
    q64, x64 = q.astype(np.float64), x.astype(np.float64)
    diff = q64[:, None, :] - x64[None, :, :]
    dot = q64 @ x64.T
    want = {
        O.L2SQ: (diff ** 2).sum(-1),
        O.L2: np.sqrt((diff ** 2).sum(-1)),
        O.COSINE: 1 - dot / (np.linalg.norm(q64, axis=1)[:, None] * np.linalg.norm(x64, axis=1)[None] + 1e-8),
        O.COSINE_NORMALIZED: 1 - dot,
        O.DOT: -dot,
        O.L1: np.abs(diff).sum(-1),
    }[metric]
    got = O.distances(q, x, metric)
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-5)


def test_sequential_order_is_the_one_written():
    # sum of (q-x)^2 in index order in fp32, no FMA: a left fold in numpy fp32
    rng = np.random.default_rng(3)
    q = rng.standard_normal(128).astype(np.float32)
    x = rng.standard_normal(128).astype(np.float32)
    s = np.float32(0)
    for a, b in zip(q, x):
        t = np.float32(a - b)
        s = np.float32(s + np.float32(t * t))
    assert O.distance(q, x, O.L2SQ) == s
    s = np.float32(0)
    for a, b in zip(q, x):
        s = np.float32(s + np.float32(abs(np.float32(a - b))))
    assert O.distance(q, x, O.L1) == s


def _brute_topk(D, k):
    # (distance, index) ascending: lexsort is a stable two-key sort
    idx = np.lexsort((np.broadcast_to(np.arange(D.shape[1]), D.shape), D), axis=1)[:, :k]
    return np.take_along_axis(D, idx, 1), idx


@pytest.mark.parametrize("metric", [O.L2SQ, O.L2, O.COSINE, O.DOT, O.L1])
def test_search_flat_is_brute_force(metric):
    rng = np.random.default_rng(10 + metric)
    q = rng.standard_normal((13, 24)).astype(np.float32)
    x = rng.standard_normal((300, 24)).astype(np.float32)
    x[7] = x[3]  # an exact tie: id 3 must come first
    q[0] = x[3]
    d, i = O.search_flat(q, x, 10, metric)
    D = O.distances(q, x, metric)
    wd, wi = _brute_topk(D, 10)
    np.testing.assert_array_equal(i, wi)
    np.testing.assert_array_equal(d, wd)
    if metric in (O.L2SQ, O.L2, O.L1):
        assert i[0, 0] == 3 and i[0, 1] == 7


def test_topk_pads_missing():
    d, i = O.topk(np.array([3, 1, 2], np.float32), 5)
    np.testing.assert_array_equal(i, [1, 2, 0, -1, -1])
    assert np.isinf(d[3:]).all()


def test_fast_variant_close():
    rng = np.random.default_rng(5)
    q = rng.standard_normal((4, 96)).astype(np.float32)
    x = rng.standard_normal((500, 96)).astype(np.float32)
    for m in (O.L2SQ, O.COSINE, O.DOT, O.L1):
        d0, i0 = O.search_flat(q, x, 5, m)
        d1, i1 = O.search_flat(q, x, 5, m, fast=True)
        np.testing.assert_allclose(d0, d1, rtol=1e-4, atol=1e-4)


def test_normalize_pinned():
    """vsko_normalize = normalizeVectors (DistanceShaders.metal:403-429):
    pinned by an explicit fp32 left fold of the squares (np.cumsum on
    float32 adds in index order), sqrt + 1e-8 in fp32 and a numpy fp32
    division per component; closed forms for a zero row (stays 0) and a
    constant row; and sensitivity: a reciprocal multiply and a pairwise
    (tree) sum each change some outputs, so this test tells them apart."""
    rng = np.random.default_rng(5)
    for n, d in ((200, 768), (300, 37), (50, 1), (64, 100)):
        x = (rng.standard_normal((n, d)) * rng.uniform(0.01, 100, (n, 1))).astype(np.float32)
        x[3] = 0.0
        got = O.normalize(x)
        sq = np.cumsum(x * x, axis=1, dtype=np.float32)[:, -1]
        m = (np.sqrt(sq, dtype=np.float32) + np.float32(1e-8)).astype(np.float32)
        want = (x / m[:, None]).astype(np.float32)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
        assert (got[3] == 0).all()
        if d >= 37:
            recip = (x * (np.float32(1) / m)[:, None]).astype(np.float32)
            assert (recip != got).any()
            tree = np.sqrt(np.sum(x * x, axis=1, dtype=np.float32)) + np.float32(1e-8)
            assert (tree.astype(np.float32) != m).any() or d < 64
    # constant row c: |x| = |c| sqrt(d) exactly for d a perfect square
    c = np.full((1, 64), 3.0, np.float32)
    np.testing.assert_array_equal(O.normalize(c), c / np.float32(np.float32(24.0) + np.float32(1e-8)))
    # unit length within rounding
    x = rng.standard_normal((100, 128)).astype(np.float32)
    assert np.allclose(np.linalg.norm(O.normalize(x).astype(np.float64), axis=1), 1.0, atol=1e-6)


def test_prepared_db_equals_search_flat():
    """O.FlatDB (the CPU baseline's resident index) returns search_flat's
    results bit for bit for every metric it serves."""
    rng = np.random.default_rng(8)
    x = rng.standard_normal((3000, 45)).astype(np.float32)
    q = rng.standard_normal((11, 45)).astype(np.float32)
    db = O.FlatDB(x)
    for metric in (O.L2SQ, O.L2, O.COSINE, O.COSINE_NORMALIZED, O.DOT, O.L1):
        a = db.search(q, 30, metric)
        b = O.search_flat(q, x, 30, metric)
        np.testing.assert_array_equal(a[0].view(np.uint32), b[0].view(np.uint32))
        np.testing.assert_array_equal(a[1], b[1])


def test_scalar_quantize_u8_pinned():
    """quantizeVectors(.scalar(bits:)) CPU path (AccelerateOptimizer.swift:
    387-430): numpy fp32 restatement (two roundings, clamp, truncation);
    closed forms: a ramp 0..255 maps to itself, a constant vector to all
    zeros with scale 1; truncation, not rounding (x = min + 0.7/scale gives
    code 0)."""
    rng = np.random.default_rng(9)
    for bits in (8, 4, 1):
        x = (rng.standard_normal((500, 37)) * rng.uniform(0.1, 50, (500, 1))).astype(np.float32)
        codes, sc, mn = O.scalar_quantize_u8(x, bits)
        emn, emx = x.min(axis=1), x.max(axis=1)
        rng_ = (emx - emn).astype(np.float32)
        es = np.where(rng_ > 0, np.float32(2 ** bits - 1) / rng_, np.float32(1)).astype(np.float32)
        t = ((x - emn[:, None]).astype(np.float32) * es[:, None]).astype(np.float32)
        want = np.clip(t, 0, 255).astype(np.uint8)  # astype truncates toward zero
        np.testing.assert_array_equal(sc, es)
        np.testing.assert_array_equal(mn, emn)
        np.testing.assert_array_equal(codes, want)
        assert codes.max() <= 2 ** bits - 1
    ramp = np.arange(256, dtype=np.float32)[None, :]
    np.testing.assert_array_equal(O.scalar_quantize_u8(ramp)[0][0], np.arange(256))
    c, s, _ = O.scalar_quantize_u8(np.full((1, 9), 2.5, np.float32))
    assert (c == 0).all() and s[0] == 1.0
    x = np.array([[0.0, 0.7, 255.0]], np.float32)
    assert O.scalar_quantize_u8(x)[0][0, 1] == 0

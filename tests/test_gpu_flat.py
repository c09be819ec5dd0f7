"""Flat k-NN on the GPU (libvsk_hip.so) against the CPU oracle.

Every metric returns the oracle's sequential fp32 distances and its
(distance, id) order bit for bit: the screened metrics (L2^2, L2, both
cosines, dot) through the bf16 screen's proven bound and the fp32 rescore,
manhattan summed in the oracle's order.  The float bar (distances within
1e-4 relative, id sets equal except for ties within that tolerance) is left
for the kernels a context selects by name (bf16x3, fp32).
"""
import numpy as np
import pytest

from oracle import oracle as O
from parity import assert_sorted_unique, assert_topk_match
from vectorstorekit_amd import VSKError, VectorDatabase
from vectorstorekit_amd._lib import (METRIC_COSINE, METRIC_COSINE_NORMALIZED, METRIC_DOT,
                                     METRIC_L1, METRIC_L2, METRIC_L2SQ)

pytestmark = pytest.mark.gpu

ALL = [METRIC_L2SQ, METRIC_L2, METRIC_COSINE, METRIC_COSINE_NORMALIZED, METRIC_DOT, METRIC_L1]


def _data(seed, n, nq, d, normalize=False):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, d)).astype(np.float32)
    q = rng.standard_normal((nq, d)).astype(np.float32)
    if normalize:
        x /= np.linalg.norm(x, axis=1, keepdims=True)
        q /= np.linalg.norm(q, axis=1, keepdims=True)
    return x, q


def _check(ctx, x, q, k, metric, exact=False):
    db = VectorDatabase(ctx, x)
    gd, gi = db.search(q, k, metric)
    od, oi = O.search_flat(q, x, k, metric)
    assert_sorted_unique(gd, gi)
    if exact:
        np.testing.assert_array_equal(gi, oi)
        np.testing.assert_array_equal(gd, od)
    else:
        assert_topk_match(gd, gi, od, oi,
                          lambda qi, ids: O.distances(q[qi:qi + 1], x[ids], metric)[0])
    return gd, gi


def test_config1_l2sq_full(ctx):
    """10,000 x 128 N(0,1), 100 queries, L2^2, k=10."""
    x, q = _data(1, 10_000, 100, 128)
    print("config1 L2SQ 10000x128 q100 k10", flush=True)
    _check(ctx, x, q, 10, METRIC_L2SQ)


@pytest.mark.parametrize("metric", ALL)
@pytest.mark.parametrize("shape", [(1000, 100, 33, 7), (5000, 70, 128, 100), (300, 3, 5, 1)])
def test_metrics_shapes(ctx, metric, shape):
    n, nq, d, k = shape
    x, q = _data(100 + metric, n, nq, d, normalize=metric == METRIC_COSINE_NORMALIZED)
    print(f"flat metric={metric} n={n} nq={nq} d={d} k={k}", flush=True)
    _check(ctx, x, q, k, metric, exact=True)


@pytest.mark.parametrize("kernel", ["bf16x3", "fp32"])
def test_named_kernels_float_bar(ctx, kernel):
    """The tolerance-path kernels a configuration selects by name (bf16x3,
    fp32 MFMA) for every metric: distances within 1e-4 relative of the
    oracle's, id sets equal except ties within that tolerance; Manhattan
    stays on the exact VALU scan (bit-exact) under either."""
    from vectorstorekit_amd.engine import Context, HIPAccelerationConfiguration

    c = Context(0, configuration=HIPAccelerationConfiguration(kernel=kernel))
    try:
        assert c.configuration().kernel == kernel
        for metric in ALL:
            x, q = _data(300 + metric, 20_000, 37, 96,
                         normalize=metric == METRIC_COSINE_NORMALIZED)
            print(f"kernel={kernel} metric={metric}", flush=True)
            _check(c, x, q, 50, metric, exact=metric == METRIC_L1)
    finally:
        c.close()


def test_chunked_path_large_n(ctx):
    """n well above the first chunk: exercises the filtered, atomic-append
    pass and the running thresholds."""
    x, q = _data(7, 200_000, 130, 64)
    print("flat chunked n=200000 nq=130 d=64 k=100", flush=True)
    _check(ctx, x, q, 100, METRIC_L2SQ)
    _check(ctx, x, q, 32, METRIC_L1, exact=True)


def test_overflow_fallback(ctx):
    """Rows get strictly closer with growing id, so every filtered chunk
    keeps everything and overflows; the sub-chunk re-scan must still give
    the exact answer."""
    n = 120_000
    x = np.zeros((n, 4), np.float32)
    x[:, 0] = np.arange(n, dtype=np.float32) / n
    q = np.array([[2.0, 0, 0, 0], [-1.0, 0, 0, 0]], np.float32)
    print("flat overflow n=120000", flush=True)
    db = VectorDatabase(ctx, x)
    gd, gi = db.search(q, 10, METRIC_L2SQ)
    od, oi = O.search_flat(q, x, 10, METRIC_L2SQ)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_allclose(gd, od, rtol=1e-4)


def test_ties_by_id(ctx):
    x, q = _data(11, 2000, 5, 16)
    x[100:110] = x[5]  # 11 identical rows
    q[:] = x[5]
    db = VectorDatabase(ctx, x)
    for metric in (METRIC_L2SQ, METRIC_L1):
        gd, gi = db.search(q, 11, metric)
        np.testing.assert_array_equal(gi[0], [5] + list(range(100, 110)))


def test_k_larger_than_n_pads(ctx):
    x, q = _data(12, 50, 4, 8)
    db = VectorDatabase(ctx, x)
    gd, gi = db.search(q, 64, METRIC_L2)
    od, oi = O.search_flat(q, x, 64, METRIC_L2)
    assert (gi[:, 50:] == -1).all() and np.isinf(gd[:, 50:]).all()
    assert_topk_match(gd, gi, od, oi, lambda qi, ids: O.distances(q[qi:qi + 1], x[ids], METRIC_L2)[0])


def test_distance_matrix(ctx):
    x, q = _data(13, 777, 9, 40)
    db = VectorDatabase(ctx, x)
    for metric in ALL:
        g = db.distances(q, metric)
        o = O.distances(q, x, metric)
        np.testing.assert_array_equal(g.view(np.uint32), o.view(np.uint32))


def test_kat_constant_rows(ctx):
    """MetalDistance512Tests.swift:50-66 / Vector512Tests.swift:174-204:
    query 0 vs rows filled with i -> sqrt(512 i^2)."""
    x = np.stack([np.full(512, i, np.float32) for i in range(100)])
    db = VectorDatabase(ctx, x)
    g = db.distances(np.zeros((1, 512), np.float32), METRIC_L2)[0]
    np.testing.assert_allclose(g, np.sqrt(512.0) * np.arange(100), rtol=1e-5, atol=1e-3)
    g1 = db.distances(np.zeros((1, 512), np.float32), METRIC_L1)[0]
    np.testing.assert_array_equal(g1, 512.0 * np.arange(100))


def test_errors(ctx):
    x, q = _data(14, 100, 3, 8)
    db = VectorDatabase(ctx, x)
    with pytest.raises(VSKError) as e:
        db.search(q, 2000, METRIC_L2)
    assert e.value.kind == "invalidBufferSize"
    with pytest.raises(VSKError) as e:
        db.search(q, 5, 42)
    assert e.value.kind == "invalidArgument"
    with pytest.raises(VSKError) as e:
        db.search(q[:0], 5, METRIC_L2)
    assert e.value.kind == "emptyInput"
    with pytest.raises(VSKError) as e:
        VectorDatabase(ctx, x[:0])
    assert e.value.kind == "emptyInput"


SCREEN = [METRIC_L2SQ, METRIC_L2, METRIC_COSINE_NORMALIZED, METRIC_DOT, METRIC_COSINE]


@pytest.fixture(scope="module")
def sctx():
    """A context that runs the screen at every size (small problems
    otherwise take the exact sequential scan alone)."""
    import os

    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from vectorstorekit_amd.engine import Context

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


@pytest.mark.parametrize("metric", SCREEN)
@pytest.mark.parametrize("shape", [(3000, 20, 128, 10), (40_000, 64, 100, 50),
                                   (20_000, 33, 37, 100), (25_000, 10, 768, 320),
                                   (6000, 12, 96, 20), (30_000, 6, 64, 700),
                                   (4000, 5, 48, 1024), (900, 3, 16, 1024)])
def test_screen_bit_exact(sctx, metric, shape):
    """The screened metrics (one-pass bf16 screen, proven bound, fp32
    rescore) return the CPU reference's sequential fp32 distances and its
    (distance, id) order exactly: one dense chunk, filtered chunks, odd d,
    k above 320 (the screen keeps VSK_MAX_K candidates, a narrower margin),
    k = VSK_MAX_K (no margin: the exact scan unless every row is kept)."""
    n, nq, d, k = shape
    x, q = _data(n + d + metric, n, nq, d, normalize=metric == METRIC_COSINE_NORMALIZED)
    print(f"screen metric={metric} n={n} nq={nq} d={d} k={k}", flush=True)
    sctx.profile(True)
    sctx.profile_reset()
    gd, gi = VectorDatabase(sctx, x).search(q, k, metric)
    stats = sctx.profile_stats()
    sctx.profile(False)
    assert "flat_screen_dense" in stats and "screen_rescore" in stats
    od, oi = O.search_flat(q, x, k, metric)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)


@pytest.mark.parametrize("metric", SCREEN)
def test_screen_fallback_near_ties(sctx, metric):
    """Rows closer to each other than the screen's error bound: the margin
    test fails for every query, at the wide second screen too, the exact
    VALU scan redoes them, and the result is still the reference's, bit for
    bit."""
    rng = np.random.default_rng(70 + metric)
    d = 64
    base = rng.standard_normal(d).astype(np.float32)
    x = (base + 1e-4 * rng.standard_normal((20_000, d))).astype(np.float32)
    q = (base + 1e-4 * rng.standard_normal((8, d))).astype(np.float32)
    if metric == METRIC_COSINE_NORMALIZED:
        x /= np.linalg.norm(x, axis=1, keepdims=True)
        q /= np.linalg.norm(q, axis=1, keepdims=True)
    print(f"screen fallback metric={metric}", flush=True)
    sctx.profile(True)
    sctx.profile_reset()
    gd, gi = VectorDatabase(sctx, x).search(q, 10, metric)
    stats = sctx.profile_stats()
    sctx.profile(False)
    assert stats["screen_retry"][2] == 8  # work counter: queries redone
    assert stats["screen_fallback"][2] == 8
    od, oi = O.search_flat(q, x, 10, metric)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)


@pytest.mark.parametrize("shape", [(1000, 768), (300, 37), (5, 1), (257, 100), (70_000, 128)])
def test_db_normalize_bit_exact(ctx, shape):
    """VSK_DB_NORMALIZE is normalizeVectors (DistanceShaders.metal:403-429):
    the stored rows equal the oracle's bit for bit (sequential sum of
    squares, sqrt + 1e-8, a division per component); zero rows stay 0;
    row counts that leave partial waves and workgroups."""
    n, d = shape
    rng = np.random.default_rng(n + d)
    x = (rng.standard_normal((n, d)) * rng.uniform(0.01, 100, (n, 1))).astype(np.float32)
    x[min(3, n - 1)] = 0.0
    db = VectorDatabase(ctx, x, normalize=True)
    want = O.normalize(x)
    np.testing.assert_array_equal(db.read().view(np.uint32), want.view(np.uint32))


def test_screen_normalized_db_and_device_queries(sctx):
    """Rows normalised on upload and queries already on the device: the
    rescore reads the stored (normalised) rows."""
    import torch

    x, q = _data(31, 30_000, 40, 96)
    db = VectorDatabase(sctx, x, normalize=True)
    xn = db.read()
    np.testing.assert_array_equal(xn, O.normalize(x))
    qn = q / np.linalg.norm(q, axis=1, keepdims=True)
    gd, gi = db.search(torch.from_numpy(qn).cuda(), 25, METRIC_COSINE_NORMALIZED)
    od, oi = O.search_flat(qn, xn, 25, METRIC_COSINE_NORMALIZED)
    np.testing.assert_array_equal(gi.cpu().numpy(), oi)
    np.testing.assert_array_equal(gd.cpu().numpy(), od)


@pytest.mark.parametrize("metric", SCREEN)
def test_small_problem_exact_scan(ctx, metric):
    """Config 1's size (at most 2^28 query x row x dimension terms) takes the
    exact sequential scan alone, without the screen, and returns the CPU
    reference's distances and order bit for bit."""
    x, q = _data(90 + metric, 10_000, 100, 128,
                 normalize=metric == METRIC_COSINE_NORMALIZED)
    print(f"small exact metric={metric}", flush=True)
    ctx.profile(True)
    ctx.profile_reset()
    gd, gi = VectorDatabase(ctx, x).search(q, 10, metric)
    stats = ctx.profile_stats()
    ctx.profile(False)
    assert "flat_screen_dense" not in stats and "screen_rescore" not in stats
    od, oi = O.search_flat(q, x, 10, metric)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)


def test_profile_only_times_the_named_kernels(ctx):
    """vsk_profile_only: with a restriction only the named timers record
    (one launch a call for the small exact scan), results unchanged; the
    restriction lifted, every kernel is timed again."""
    x, q = _data(7, 10_000, 100, 128)
    db = VectorDatabase(ctx, x)
    ctx.profile(True)
    ctx.profile_only(["flat_valu_dense"])
    ctx.profile_reset()
    gd, gi = db.search(q, 10, METRIC_L2)
    stats = ctx.profile_stats()
    assert list(stats) == ["flat_valu_dense"] and stats["flat_valu_dense"][0] == 1
    ctx.profile_only(None)
    ctx.profile_reset()
    gd2, gi2 = db.search(q, 10, METRIC_L2)
    stats = ctx.profile_stats()
    ctx.profile(False)
    assert "flat_valu_dense" in stats and "flat_select" in stats
    np.testing.assert_array_equal(gi, gi2)
    np.testing.assert_array_equal(gd, gd2)


def test_upload_read_roundtrip_padded_chunked(ctx):
    """Host rows with a pitch that needs padding (d=129 -> 132) and more than
    one 64 MB staging chunk: upload and read-back are exact, from host and
    from device memory, and a row window reads back the same rows."""
    import torch

    rng = np.random.default_rng(21)
    x = rng.standard_normal((140_000, 129)).astype(np.float32)
    db = VectorDatabase(ctx, x)
    np.testing.assert_array_equal(db.read(), x)
    np.testing.assert_array_equal(db.read(70_001, 1234), x[70_001:71_235])
    db.free()
    xd = torch.from_numpy(x[:5000]).cuda()
    db = VectorDatabase(ctx, xd)
    np.testing.assert_array_equal(db.read(), x[:5000])
    db.free()
    # narrow rows (8 floats) from host: the IVF assign staging path
    xs = rng.standard_normal((65_536, 8)).astype(np.float32)
    db = VectorDatabase(ctx, xs)
    np.testing.assert_array_equal(db.read(), xs)
    db.free()


def test_device_tensors(ctx):
    """Inputs/outputs as torch device tensors take the zero-copy path."""
    import torch

    x, q = _data(15, 3000, 17, 64)
    xt, qt = torch.from_numpy(x).cuda(), torch.from_numpy(q).cuda()
    db = VectorDatabase(ctx, xt)
    gd, gi = db.search(qt, 20, METRIC_COSINE)
    assert gd.is_cuda and gi.is_cuda
    hd, hi = VectorDatabase(ctx, x).search(q, 20, METRIC_COSINE)
    np.testing.assert_array_equal(gi.cpu().numpy(), hi)
    np.testing.assert_array_equal(gd.cpu().numpy(), hd)


def test_config2_cosine_full_size(ctx):
    """BASELINE config 2 at full size: 1,000,000 x 768 unit-norm rows, 10,000
    queries, k = 100.  Bit-exact against the oracle (distances bit for bit,
    ids equal) on all 10,000 queries; the queries the screen redid (tier 1:
    the wider screen; tier 2: the exact scan) must number as the
    screen_retry / screen_fallback work counters say (printed: none on this
    data)."""
    import torch

    n, d, nq, k = 1_000_000, 768, 10_000, 100
    g = torch.Generator(device="cuda")
    g.manual_seed(1)
    x = torch.randn(n, d, generator=g, device="cuda")
    x /= x.norm(dim=1, keepdim=True)
    g.manual_seed(2)
    q = torch.randn(nq, d, generator=g, device="cuda")
    q /= q.norm(dim=1, keepdim=True)
    print("config2 cosine 1Mx768 q10000 k100", flush=True)
    db = VectorDatabase(ctx, x)
    ctx.profile(True)
    ctx.profile_reset()
    try:
        gd, gi = db.search(q, k, METRIC_COSINE_NORMALIZED)
        stats = ctx.profile_stats()
    finally:
        ctx.profile(False)
    assert stats["flat_screen_filter"][0] > 0  # the bf16 screen path ran
    tier1, tier2 = ctx.last_screen_redo(1), ctx.last_screen_redo(2)
    assert len(tier1) == int(stats.get("screen_retry", (0, 0, 0))[2])
    assert len(tier2) == int(stats.get("screen_fallback", (0, 0, 0))[2])
    print(f"screen redo: {len(tier1)} queries in tier 1, {len(tier2)} in tier 2", flush=True)
    gd, gi = gd.cpu().numpy(), gi.cpu().numpy()
    assert_sorted_unique(gd, gi)
    assert (gi >= 0).all() and (gi < n).all()
    xh, qh = x.cpu().numpy(), q.cpu().numpy()
    del x
    od, oi = O.search_flat(qh, xh, k, METRIC_COSINE_NORMALIZED)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd.view(np.uint32), od.view(np.uint32))
    # the distances are 1 - q.x of the returned rows within fp32 rounding
    # (each row a unit vector)
    some = np.random.default_rng(0).choice(nq, 64, replace=False)
    for qi in some:
        ref = 1.0 - xh[gi[qi]].astype(np.float64) @ qh[qi].astype(np.float64)
        np.testing.assert_allclose(gd[qi], ref, rtol=0, atol=2e-6)


def test_config2_planted_near_ties(ctx):
    """Config 2's database and queries with near-duplicate clusters planted
    around three queries: 600 rows (more than the 364 the screen keeps, fewer
    than the 1,024 of its second tier) around query 0 and 1,600 rows (more
    than both) around queries 1 and 2, all within the screen's error bound of
    each other.  Those queries fail the bound: query 0 is settled by the
    wider screen (tier 1), queries 1 and 2 by the exact scan over every row
    (tier 2).  All 10,000 queries bit-exact against the oracle."""
    import torch

    n, d, nq, k = 1_000_000, 768, 10_000, 100
    g = torch.Generator(device="cuda")
    g.manual_seed(1)
    x = torch.randn(n, d, generator=g, device="cuda")
    x /= x.norm(dim=1, keepdim=True)
    g.manual_seed(2)
    q = torch.randn(nq, d, generator=g, device="cuda")
    q /= q.norm(dim=1, keepdim=True)
    g.manual_seed(9)
    at = 0
    for qi, m in ((0, 600), (1, 1600), (2, 1600)):
        rows = q[qi] + 0.01 * torch.randn(m, d, generator=g, device="cuda")
        x[at:at + m] = rows / rows.norm(dim=1, keepdim=True)
        at += m
    print("config2 planted near ties 1Mx768 q10000 k100", flush=True)
    db = VectorDatabase(ctx, x)
    gd, gi = db.search(q, k, METRIC_COSINE_NORMALIZED)
    tier1, tier2 = ctx.last_screen_redo(1), ctx.last_screen_redo(2)
    print(f"screen redo: tier 1 {tier1.tolist()[:10]} ({len(tier1)}), "
          f"tier 2 {tier2.tolist()[:10]} ({len(tier2)})", flush=True)
    assert {0, 1, 2} <= set(tier1.tolist())
    assert {1, 2} <= set(tier2.tolist()) and 0 not in set(tier2.tolist())
    gd, gi = gd.cpu().numpy(), gi.cpu().numpy()
    xh, qh = x.cpu().numpy(), q.cpu().numpy()
    del x
    od, oi = O.search_flat(qh, xh, k, METRIC_COSINE_NORMALIZED)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd.view(np.uint32), od.view(np.uint32))
    assert set(gi[1].tolist()) <= set(range(600, 2200))


def test_config2_scale_epsilon_cosine(ctx):
    """The reference's epsilon cosine (1 - q.x / (|q||x| + 1e-8)) at config
    2's scale on rows of varied norm (not normalised): 400,000 x 768, 2,000
    queries, k = 100, through the bf16 screen with the relative bound and
    the fp32 rescore; a zero query (distance 1 to every row, ties by id) and
    a zero row.  Bit-exact against the oracle."""
    import torch

    n, d, nq, k = 400_000, 768, 2_000, 100
    g = torch.Generator(device="cuda")
    g.manual_seed(21)
    x = torch.randn(n, d, generator=g, device="cuda")
    x *= torch.rand(n, 1, generator=g, device="cuda") * 50 + 0.01
    x[7] = 0.0
    g.manual_seed(22)
    q = torch.randn(nq, d, generator=g, device="cuda") * 3.0
    q[5] = 0.0
    print("config2-scale epsilon cosine 400000x768 q2000 k100", flush=True)
    db = VectorDatabase(ctx, x)
    ctx.profile(True)
    ctx.profile_reset()
    try:
        gd, gi = db.search(q, k, METRIC_COSINE)
        stats = ctx.profile_stats()
    finally:
        ctx.profile(False)
    assert stats["flat_screen_filter"][0] > 0  # the bf16 screen path ran
    print(f"screen redo: tier 1 {len(ctx.last_screen_redo(1))}, "
          f"tier 2 {len(ctx.last_screen_redo(2))}", flush=True)
    gd, gi = gd.cpu().numpy(), gi.cpu().numpy()
    xh, qh = x.cpu().numpy(), q.cpu().numpy()
    del x
    od, oi = O.search_flat(qh, xh, k, METRIC_COSINE)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd.view(np.uint32), od.view(np.uint32))
    np.testing.assert_array_equal(gi[5], np.arange(k))
    assert (gd[5] == 1.0).all()


@pytest.mark.parametrize("metric", ["euclidean", "manhattan", "cosine", "hamming"])
def test_distance_matrix_symmetric(ctx, metric):
    """computeDistanceMatrix(vectorsA) is the symmetric matrix of A: equal to
    its transpose bit for bit, a zero diagonal for the distance metrics, and
    the oracle's values bit for bit."""
    from vectorstorekit_amd import HIPAccelerationEngine

    rng = np.random.default_rng(3)
    a = rng.standard_normal((700, 45)).astype(np.float32)
    if metric == "hamming":
        a = rng.integers(0, 3, (700, 45)).astype(np.float32)
    eng = HIPAccelerationEngine(ctx)
    m = np.asarray(eng.computeDistanceMatrix(a, metric=metric))
    np.testing.assert_array_equal(m, m.T)
    code = {"euclidean": O.L2, "manhattan": O.L1, "cosine": O.COSINE, "hamming": O.HAMMING}[metric]
    ref = O.distances(a, a, code)
    np.testing.assert_array_equal(m.view(np.uint32), ref.view(np.uint32))
    if metric != "cosine":
        assert (np.diag(m) == 0).all()
    b = rng.standard_normal((33, 45)).astype(np.float32)
    mb = np.asarray(eng.computeDistanceMatrix(b, a, metric="manhattan"))
    np.testing.assert_array_equal(mb, O.distances(b, a, O.L1))


@pytest.mark.parametrize("metric", [METRIC_L2SQ, METRIC_L2, METRIC_COSINE_NORMALIZED,
                                    METRIC_DOT, METRIC_L1, METRIC_COSINE])
@pytest.mark.parametrize("shape", [(20_000, 64, 96, 10, 0.005), (5000, 40, 37, 100, 0.4),
                                   (3000, 300, 768, 50, 0.05), (120_000, 100, 128, 100, 0.5)])
def test_flat_filtered(ctx, metric, shape):
    """vsk_search_flat_filtered: the search over the rows the filter keeps,
    with their own row ids -- bit-exact against the oracle over those rows,
    as the unfiltered search; a filter as allowed ids with a short bitmap;
    nothing allowed."""
    n, nq, d, k, frac = shape
    x, q = _data(7 * n + metric, n, nq, d, normalize=metric == METRIC_COSINE_NORMALIZED)
    print(f"flat filter metric={metric} n={n} nq={nq} d={d} k={k} keep={frac}", flush=True)
    db = VectorDatabase(ctx, x)
    keep = np.random.default_rng(n + k).random(n) < frac
    sub = np.flatnonzero(keep)
    gd, gi = db.search(q, k, metric, allow=keep)
    od, oi = O.search_flat(q, x[sub], k, metric)
    oi = np.where(oi >= 0, sub[np.maximum(oi, 0)], -1)
    assert_sorted_unique(gd, gi)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)
    assert set(gi[gi >= 0].tolist()) <= set(sub.tolist())
    # allowed ids with a bitmap of n // 2 bits: the rows past it are out
    ids = sub[sub < n // 2]
    gd2, gi2 = db.search(q, k, metric, allow=ids)
    od2, oi2 = O.search_flat(q, x[ids], k, metric)
    oi2 = np.where(oi2 >= 0, ids[np.maximum(oi2, 0)], -1)
    np.testing.assert_array_equal(gi2, oi2)
    np.testing.assert_array_equal(gd2, od2)
    gd3, gi3 = db.search(q[:2], k, metric, allow=np.zeros(n, np.bool_))
    assert (gi3 == -1).all() and np.isinf(gd3).all()


def test_screen_segment_overflow_rescan(ctx):
    """A filtered chunk of the screen whose survivors overflow a query's
    per-split segment: 900 near-copies of query 0 placed after the first
    dense chunk (2,048 rows) all beat its running threshold, more than a
    split's segment holds.  The call notices at its end and runs again with
    a check per chunk; the overflowing query re-scans that chunk in dense
    sub-chunks, whose keys the selection must read as dense lists (not in
    the filtered chunk's segmented layout).  Bit-exact for every query."""
    import os

    from vectorstorekit_amd import Context

    rng = np.random.default_rng(41)
    n, nq, d, k = 60_000, 300, 64, 100
    x = rng.standard_normal((n, d)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    q = rng.standard_normal((nq, d)).astype(np.float32)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    near = q[0] + 0.05 * rng.standard_normal((900, d)).astype(np.float32)
    x[3000:3900] = near / np.linalg.norm(near, axis=1, keepdims=True)
    old = os.environ.get("VSK_FLAT_KERNEL")
    os.environ["VSK_FLAT_KERNEL"] = "screen"
    try:
        sctx = Context(0)
    finally:
        if old is None:
            del os.environ["VSK_FLAT_KERNEL"]
        else:
            os.environ["VSK_FLAT_KERNEL"] = old
    db = VectorDatabase(sctx, x)
    gd, gi = db.search(q, k, METRIC_COSINE_NORMALIZED)
    waits = sctx.last_sync_count()
    od, oi = O.search_flat(q, x, k, METRIC_COSINE_NORMALIZED)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)
    print(f"segment overflow: {waits} host waits", flush=True)
    assert waits > 2, "no chunk overflowed"
    db.free()
    sctx.close()


def test_epsilon_cosine_rows_outside_the_bound(sctx):
    """Rows the epsilon-cosine screen's relative bound cannot cover: a row
    whose squares underflow (norm 0 in fp32, components not zero) and a row
    of norm above 2^60.  The database then takes the exact scan, bit for bit
    the oracle's; a database without them takes the screen again.  (Rows
    with non-finite components are refused by the same test, but their NaN
    distances have no order the oracle's heap keeps, so no parity is
    claimed for them.)"""
    rng = np.random.default_rng(55)
    x = rng.standard_normal((6000, 48)).astype(np.float32)
    q = rng.standard_normal((9, 48)).astype(np.float32)
    x[10] = 1e-30
    x[11] = 3e18
    print("cosine rows outside the bound", flush=True)
    sctx.profile(True)
    sctx.profile_reset()
    gd, gi = VectorDatabase(sctx, x).search(q, 40, METRIC_COSINE)
    stats = sctx.profile_stats()
    sctx.profile(False)
    assert "flat_screen_dense" not in stats and "screen_rescore" not in stats
    od, oi = O.search_flat(q, x, 40, METRIC_COSINE)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd.view(np.uint32), od.view(np.uint32))
    # the same rows without the two: the screen runs, still exact
    y = np.delete(x, [10, 11], axis=0)
    sctx.profile(True)
    sctx.profile_reset()
    gd, gi = VectorDatabase(sctx, y).search(q, 40, METRIC_COSINE)
    stats = sctx.profile_stats()
    sctx.profile(False)
    assert "screen_rescore" in stats
    od, oi = O.search_flat(q, y, 40, METRIC_COSINE)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd.view(np.uint32), od.view(np.uint32))

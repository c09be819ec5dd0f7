"""The engine mirror through the C ABI: HIPAcceleratorStrategy.capabilities
(vsk_device_info), HIPAccelerationEngine.computeDistances /
batchComputeDistances(topK:) / quantizeVectors, vsk_last_kernel_ms, and
that per-call candidate uploads are freed."""
import numpy as np
import pytest

from oracle import oracle as O
from vectorstorekit_amd import (Context, HIPAccelerationEngine, HIPAcceleratorStrategy,
                                QuantizationParameters, QuantizationScheme, VectorDatabase,
                                VSKError)

pytestmark = pytest.mark.gpu


def test_capabilities_and_strategy(ctx):
    s = HIPAcceleratorStrategy(0)
    c = s.capabilities()
    assert s.initialize() is s.initialize()
    assert c["arch"].startswith("gfx950")
    assert c["wavefront_size"] == 64
    assert c["compute_units"] >= 256
    assert c["global_mem_bytes"] > 200 * 2 ** 30
    assert c["lds_bytes_per_block"] >= 64 * 1024
    s.initialize().close()


@pytest.mark.parametrize("metric,code", [("euclidean", O.L2), ("manhattan", O.L1),
                                         ("euclideanSquared", O.L2SQ), ("hamming", O.HAMMING)])
def test_compute_distances_exact(ctx, metric, code):
    """computeDistances(query:candidates:metric:) for one query: the exact
    metrics are the oracle's sums bit for bit."""
    rng = np.random.default_rng(1)
    cand = rng.standard_normal((3000, 45)).astype(np.float32)
    q = rng.standard_normal(45).astype(np.float32)
    if metric == "hamming":
        cand = rng.integers(0, 3, (3000, 45)).astype(np.float32)
        q = rng.integers(0, 3, 45).astype(np.float32)
    eng = HIPAccelerationEngine(ctx)
    got = np.asarray(eng.computeDistances(q, cand, metric))
    np.testing.assert_array_equal(got, O.distances(q[None], cand, code)[0])
    assert ctx.last_kernel_ms > 0.0


@pytest.mark.parametrize("metric,code", [("cosine", O.COSINE), ("dotProduct", O.DOT)])
def test_compute_distances_cosine_dot_exact(ctx, metric, code):
    """cosine (the reference's epsilon form) and dot: the oracle's
    sequential fp32 values bit for bit."""
    rng = np.random.default_rng(2)
    cand = rng.standard_normal((2000, 64)).astype(np.float32)
    q = rng.standard_normal(64).astype(np.float32)
    got = np.asarray(HIPAccelerationEngine(ctx).computeDistances(q, cand, metric))
    want = O.distances(q[None], cand, code)[0]
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_batch_compute_distances(ctx):
    """batchComputeDistances(queries:candidates:metric:topK:): the full
    matrix without topK, the k smallest per query (ascending) with it; a
    topK above the candidate count returns every candidate."""
    rng = np.random.default_rng(3)
    cand = rng.standard_normal((5000, 33)).astype(np.float32)
    qs = rng.standard_normal((7, 33)).astype(np.float32)
    eng = HIPAccelerationEngine(ctx)
    full = np.asarray(eng.batchComputeDistances(qs, cand, "euclidean"))
    np.testing.assert_array_equal(full, O.distances(qs, cand, O.L2))
    top = np.asarray(eng.batchComputeDistances(qs, cand, "euclidean", topK=25))
    od, _ = O.search_flat(qs, cand, 25, O.L2)
    np.testing.assert_array_equal(top, od)
    small = np.asarray(eng.batchComputeDistances(qs, cand[:10], "manhattan", topK=50))
    assert small.shape == (7, 10)
    np.testing.assert_array_equal(small, np.sort(O.distances(qs, cand[:10], O.L1), axis=1))
    # a resident database is used as is
    db = VectorDatabase(ctx, cand)
    np.testing.assert_array_equal(np.asarray(eng.batchComputeDistances(qs, db, "euclidean",
                                                                       topK=25)), od)
    with pytest.raises(VSKError):
        eng.computeDistances(qs[0], np.empty((0, 33), np.float32))


def test_per_call_uploads_are_freed(ctx):
    """Candidates passed as arrays are uploaded for the call and freed: 40
    calls on 64 MB of candidates leave device memory where it was."""
    import torch

    rng = np.random.default_rng(4)
    cand = rng.standard_normal((250_000, 64)).astype(np.float32)
    q = rng.standard_normal((2, 64)).astype(np.float32)
    eng = HIPAccelerationEngine(ctx)
    eng.batchComputeDistances(q, cand, "euclidean", topK=10)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(20):
        eng.batchComputeDistances(q, cand, "euclidean", topK=10)
        eng.computeDistances(q[0], cand, "manhattan")
    torch.cuda.synchronize()
    assert free0 - torch.cuda.mem_get_info()[0] < 256 * 2 ** 20


@pytest.mark.parametrize("bits", [8, 4])
def test_quantize_vectors_scalar(ctx, bits):
    """quantizeVectors(scheme: .scalar(bits:)): per-vector min/max codes,
    scale and minimum bit for bit against the oracle's restatement."""
    rng = np.random.default_rng(5 + bits)
    x = (rng.standard_normal((3000, 77)) * rng.uniform(0.1, 30, (3000, 1))).astype(np.float32)
    x[10] = 1.5  # a constant vector: scale 1, codes 0
    qv = HIPAccelerationEngine(ctx).quantizeVectors(x, QuantizationScheme.scalar(bits))
    codes = np.stack([np.frombuffer(v.codes, np.uint8) for v in qv])
    ec, es, em = O.scalar_quantize_u8(x, bits)
    np.testing.assert_array_equal(codes, ec)
    np.testing.assert_array_equal(np.array([v.scale for v in qv], np.float32), es)
    np.testing.assert_array_equal(np.array([v.minimum for v in qv], np.float32), em)
    assert qv[0].originalDimensions == 77 and qv[0].scheme.kind == "scalar"
    assert qv[0].metadata.compressionRatio == pytest.approx(77 * 4 / 85)


def test_quantize_vectors_binary_product_none(ctx):
    import torch

    rng = np.random.default_rng(6)
    x = rng.standard_normal((2000, 32)).astype(np.float32)
    eng = HIPAccelerationEngine(ctx)
    qb = eng.quantizeVectors(x, QuantizationScheme.binary())
    codes = np.stack([np.frombuffer(v.codes, np.uint8) for v in qb])
    np.testing.assert_array_equal(codes, O.binary_encode(x))
    # product: k-means codebooks per segment, one byte per segment; the
    # same as training and encoding with ProductQuantizer directly
    from vectorstorekit_amd import ProductQuantizer

    params = QuantizationParameters(trainingIterations=5, seed=3)
    qp = eng.quantizeVectors(torch.from_numpy(x).cuda(), QuantizationScheme.product(4, 6), params)
    pc = np.stack([np.frombuffer(v.codes, np.uint8) for v in qp])
    pq = ProductQuantizer.train(ctx, x, 4, 64, iterations=5, seed=3)
    np.testing.assert_array_equal(pc, pq.encode(x))
    np.testing.assert_array_equal(pc, O.pq_encode(x, pq.codebooks))
    assert pc.shape == (2000, 4) and pc.max() < 64
    raw = eng.quantizeVectors(x[:3], QuantizationScheme.none())
    assert raw[1].codes == x[1].tobytes() and raw[1].metadata.compressionRatio == 1.0
    with pytest.raises(VSKError):
        eng.quantizeVectors(x, QuantizationScheme.product(5))


@pytest.mark.gpu
def test_measure_peaks_plausible():
    """vsk_measure_peaks: each ceiling is positive and within a factor of
    the MI355X datasheet figure (bf16 2.5 PFLOP/s, int8 5.0 POP/s, HBM
    8 TB/s); a measured rate above 1.1x the datasheet would mean the timing
    or the operation count is wrong."""
    ctx = Context(0)
    try:
        pk = ctx.measure_peaks()
    finally:
        ctx.close()
    for key, sheet in (("bf16_tflops", 2500.0), ("int8_tops", 5000.0), ("hbm_gbs", 8000.0),
                       ("hbm_read_gbs", 8000.0)):
        assert 0.25 * sheet < pk[key] < 1.1 * sheet, (key, pk[key])


def test_matrix_multiply_bit_exact(ctx):
    """matrixMultiply (MetalAccelerationEngine.swift:209-229): the
    reference test's known answer (MetalComponentTests.swift:244-271), then
    ragged shapes (partial tiles in every dimension, k past one inner step,
    single rows and columns) and device tensors, each entry the oracle's
    in-order sum bit for bit; a dimension mismatch and an empty matrix
    raise."""
    import json
    import os

    eng = HIPAccelerationEngine(ctx)
    kat = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                      "reference_kats.json")))["matrix_multiply"]
    c = np.asarray(eng.matrixMultiply(kat["a"], kat["b"]))
    np.testing.assert_array_equal(c, np.array(kat["c"], np.float32))
    rng = np.random.default_rng(11)
    for m, k, n in ((1, 1, 1), (67, 33, 130), (64, 32, 64), (5, 1000, 3), (300, 768, 257)):
        a = rng.standard_normal((m, k)).astype(np.float32)
        b = rng.standard_normal((k, n)).astype(np.float32)
        print(f"matmul {m}x{k}x{n}", flush=True)
        got = np.asarray(eng.matrixMultiply(a, b))
        np.testing.assert_array_equal(got.view(np.uint32), O.matmul(a, b).view(np.uint32))
    import torch

    a = rng.standard_normal((129, 70)).astype(np.float32)
    b = rng.standard_normal((70, 65)).astype(np.float32)
    got = eng.matrixMultiply(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda())
    assert got.is_cuda
    np.testing.assert_array_equal(got.cpu().numpy(), O.matmul(a, b))
    with pytest.raises(VSKError):
        eng.matrixMultiply(a, a)
    with pytest.raises(VSKError):
        eng.matrixMultiply(np.empty((0, 4), np.float32), np.ones((4, 2), np.float32))

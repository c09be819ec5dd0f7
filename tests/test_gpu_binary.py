"""Binary quantization, the Hamming top-k scan and the float hamming metric
on the GPU against the oracle: all integer (or integer-valued) results,
held bit-exact."""
import numpy as np
import pytest

from oracle import oracle as O
from parity import assert_sorted_unique
from vectorstorekit_amd import BinaryDatabase, BinaryQuantizer, VectorDatabase, VSKError
from vectorstorekit_amd._lib import METRIC_HAMMING

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("d", [1, 7, 8, 37, 128, 1000, 1024])
def test_binary_encode_bit_exact(ctx, d):
    rng = np.random.default_rng(d)
    x = rng.standard_normal((3001, d)).astype(np.float32)
    x[0] = 0.0
    x[1, ::2] = -0.0
    np.testing.assert_array_equal(BinaryQuantizer(ctx).quantizeBatch(x), O.binary_encode(x))


@pytest.mark.parametrize("shape", [(50_000, 128, 37, 100), (3000, 37, 50, 10),
                                   (20_000, 1024, 9, 1024), (100, 64, 5, 300),
                                   (200_000, 256, 70, 20), (9_000, 500, 33, 1),
                                   (12_000, 1000, 40, 64), (30_001, 130, 16, 100),
                                   (5_003, 96, 600, 7)])
def test_bin_search_bit_exact(ctx, shape):
    """Code widths of 4, 8, 16 and 32 words (d = 37 .. 1024), k = 1 .. 1024,
    k > n (padding), several chunks of the progressive scan, partial row
    groups (n = 5,003, 30,001), a partial query tile (16 and 600 queries on
    the int8 matrix-core scan; under 16 on the popcount scan); distances and
    ids equal the oracle's (distance, id) order despite the large ties of
    integer distances."""
    n, d, nq, k = shape
    print(f"bin search n={n} d={d} nq={nq} k={k}", flush=True)
    rng = np.random.default_rng(n + d)
    x = rng.standard_normal((n, d)).astype(np.float32)
    q = rng.standard_normal((nq, d)).astype(np.float32)
    xc, qc = O.binary_encode(x), O.binary_encode(q)
    xc[7] = xc[3]  # a duplicate row: equal distances, the lower id first
    db = BinaryDatabase(ctx, xc, d)
    gd, gi = db.search(qc, k)
    od, oi = O.bin_search(qc, xc, d, k)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)
    db.free()


def test_bin_distances_matrix(ctx):
    rng = np.random.default_rng(5)
    d = 100
    xc = O.binary_encode(rng.standard_normal((5000, d)).astype(np.float32))
    qc = O.binary_encode(rng.standard_normal((13, d)).astype(np.float32))
    db = BinaryDatabase(ctx, xc, d)
    m = db.distances(qc)
    ux = np.unpackbits(xc, axis=1, bitorder="little")[:, :d]
    uq = np.unpackbits(qc, axis=1, bitorder="little")[:, :d]
    np.testing.assert_array_equal(m, (uq[:, None, :] != ux[None]).sum(-1).astype(np.float32))


def test_bin_device_tensors_and_errors(ctx):
    import torch

    rng = np.random.default_rng(6)
    x = rng.standard_normal((10_000, 64)).astype(np.float32)
    xt = torch.from_numpy(x).cuda()
    codes = BinaryQuantizer(ctx).quantizeBatch(xt)
    assert codes.is_cuda
    np.testing.assert_array_equal(codes.cpu().numpy(), O.binary_encode(x))
    db = BinaryDatabase(ctx, codes, 64)
    d, i = db.search(codes[:10], 5)
    assert d.is_cuda and (d[:, 0] == 0).all().item()
    with pytest.raises(VSKError) as e:
        BinaryDatabase(ctx, np.zeros((10, 129), np.uint8), 1030)
    assert e.value.kind == "unsupportedOperation"
    with pytest.raises(VSKError) as e:
        db.search(codes[:2], 2000)
    assert e.value.kind == "invalidBufferSize"


@pytest.mark.parametrize("shape", [(20_000, 40, 17, 50), (3000, 7, 9, 10)])
def test_flat_hamming_metric_bit_exact(ctx, shape):
    """DistanceMetric.hamming on float rows: the count of unequal components
    (small integer data so that many components match), top-k and matrix."""
    n, d, nq, k = shape
    rng = np.random.default_rng(n)
    x = rng.integers(0, 3, (n, d)).astype(np.float32)
    q = rng.integers(0, 3, (nq, d)).astype(np.float32)
    db = VectorDatabase(ctx, x)
    gd, gi = db.search(q, k, "hamming")
    od, oi = O.search_flat(q, x, k, O.HAMMING)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)
    assert_sorted_unique(gd, gi)
    np.testing.assert_array_equal(db.distances(q[:3], "hamming"), O.distances(q[:3], x, O.HAMMING))


def test_config4_binary_full_size(ctx):
    """Binary codes of config 4's data (10M x 128 N(0,1) rows -> 16 bytes
    each), 1,000 queries, k = 100: encoded on the GPU, searched, and 32
    queries checked bit-exact against the oracle over all 10M rows."""
    import torch

    n, d, nq, k = 10_000_000, 128, 1000, 100
    g = torch.Generator(device="cuda")
    g.manual_seed(1)
    x = torch.randn(n, d, generator=g, device="cuda")
    g.manual_seed(2)
    q = torch.randn(nq, d, generator=g, device="cuda")
    print("config4 binary 10Mx128 q1000 k100", flush=True)
    bq = BinaryQuantizer(ctx)
    xc, qc = bq.quantizeBatch(x), bq.quantizeBatch(q)
    del x
    db = BinaryDatabase(ctx, xc, d)
    gd, gi = db.search(qc, k)
    xh, qh = xc.cpu().numpy(), qc.cpu().numpy()
    np.testing.assert_array_equal(xh[:1000], O.binary_encode(torch.randn(
        n, d, generator=g.manual_seed(1), device="cuda")[:1000].cpu().numpy()))
    od, oi = O.bin_search(qh[:32], xh, d, k)
    np.testing.assert_array_equal(gi.cpu().numpy()[:32], oi)
    np.testing.assert_array_equal(gd.cpu().numpy()[:32], od)

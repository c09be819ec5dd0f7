"""Batched HNSW neighbour distances (vsk_hnsw_distances) and the lockstep
layer-0 search built on them, against the oracle: DistanceComputer's
distances bit for bit (Indexes/HNSWIndex.swift:1920-1959) and
searchLayer0's results (:1151-1212) equal."""
import numpy as np
import pytest

from oracle import oracle as O
from vectorstorekit_amd import VectorDatabase, VSKError
from vectorstorekit_amd.hnsw import HNSWBatchSearch, neighbor_distances

pytestmark = pytest.mark.gpu

METRICS = [("euclidean", O.L2), ("euclideanSquared", O.L2SQ), ("manhattan", O.L1),
           ("cosine", O.COSINE_NOEPS)]


def _csr(rng, nq, n, max_deg, empty_every=7):
    counts = rng.integers(0, max_deg + 1, nq)
    counts[::empty_every] = 0
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    rows = rng.integers(0, n, int(off[-1])).astype(np.int32)
    return off, rows


@pytest.mark.parametrize("shape", [(5000, 128, 300, 48), (3000, 37, 77, 20), (900, 3, 40, 9),
                                   (2000, 200, 129, 100)])
@pytest.mark.parametrize("metric,code", METRICS)
def test_hnsw_distances_bit_exact(ctx, shape, metric, code):
    n, d, nq, deg = shape
    print(f"hnsw n={n} d={d} nq={nq} deg={deg} {metric}", flush=True)
    rng = np.random.default_rng(n + d + code)
    x = rng.standard_normal((n, d)).astype(np.float32)
    q = rng.standard_normal((nq, d)).astype(np.float32)
    off, rows = _csr(rng, nq, n, deg)
    db = VectorDatabase(ctx, x)
    got = np.asarray(neighbor_distances(db, q, off, rows, metric))
    want = O.hnsw_distances(q, x, off, rows, code)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_hnsw_cosine_zero_vector_and_device_tensors(ctx):
    """No epsilon: a zero row gives NaN, as the reference's division 0/0;
    device inputs and outputs stay on the device."""
    import torch

    rng = np.random.default_rng(9)
    x = rng.standard_normal((300, 16)).astype(np.float32)
    x[7] = 0
    q = rng.standard_normal((3, 16)).astype(np.float32)
    off = np.array([0, 2, 2, 5], np.int64)
    rows = np.array([7, 1, 2, 7, 299], np.int32)
    db = VectorDatabase(ctx, x)
    got = neighbor_distances(db, torch.from_numpy(q).cuda(), torch.from_numpy(off).cuda(),
                             torch.from_numpy(rows).cuda(), "cosine")
    assert got.is_cuda
    got = got.cpu().numpy()
    want = O.hnsw_distances(q, x, off, rows, O.COSINE_NOEPS)
    np.testing.assert_array_equal(got, want)  # NaN where the row is zero
    assert np.isnan(got[0]) and np.isnan(got[3]) and not np.isnan(got[2])


def test_hnsw_errors(ctx):
    rng = np.random.default_rng(10)
    x = rng.standard_normal((100, 8)).astype(np.float32)
    db = VectorDatabase(ctx, x)
    q = rng.standard_normal((2, 8)).astype(np.float32)
    with pytest.raises(VSKError) as e:
        neighbor_distances(db, q, np.array([0, 1, 2], np.int64), np.array([3, 100], np.int32))
    assert e.value.status == -2
    with pytest.raises(VSKError) as e:
        neighbor_distances(db, q, np.array([0, 2, 1], np.int64), np.array([3], np.int32))
    assert e.value.status == -2
    with pytest.raises(VSKError) as e:
        neighbor_distances(db, q, np.array([0, 1, 2], np.int64), np.array([3, 4], np.int32), 4)
    assert e.value.status == -8
    assert len(neighbor_distances(db, q, np.zeros(3, np.int64), np.zeros(0, np.int32))) == 0


def _graph(rng, x, deg):
    """A small navigable graph: each node's deg/2 nearest nodes plus deg/2
    random ones."""
    n = x.shape[0]
    d2 = ((x[:, None, :].astype(np.float64) - x[None, :, :]) ** 2).sum(-1)
    np.fill_diagonal(d2, np.inf)
    near = np.argsort(d2, axis=1)[:, :deg // 2]
    far = rng.integers(0, n, (n, deg // 2))
    return [list(dict.fromkeys([int(v) for v in near[i]] + [int(v) for v in far[i] if v != i]))
            for i in range(n)]


@pytest.mark.parametrize("metric,code", [("euclidean", O.L2), ("cosine", O.COSINE_NOEPS),
                                         ("manhattan", O.L1)])
def test_batch_search_layer0_equals_sequential(ctx, metric, code):
    """The lockstep batch search returns, for every query, exactly the
    sequential searchLayer0's (distance, node) list; deleted nodes skipped."""
    rng = np.random.default_rng(11 + code)
    n, d, nq, ef = 1500, 24, 40, 16
    x = rng.standard_normal((n, d)).astype(np.float32)
    q = rng.standard_normal((nq, d)).astype(np.float32)
    adj = _graph(rng, x, 16)
    deleted = set(rng.choice(n, 30, replace=False).tolist()) - {0}
    entries = rng.integers(0, n, nq)
    entries = [int(e) if int(e) not in deleted else 0 for e in entries]
    db = VectorDatabase(ctx, x)
    bs = HNSWBatchSearch(db, adj, metric, deleted=deleted)
    got = bs.search_layer0(q, entries, ef)
    for i in range(nq):
        want = O.search_layer0(q[i], x, adj, entries[i], ef, code, deleted=deleted)
        assert [t[1] for t in got[i]] == [t[1] for t in want]
        np.testing.assert_array_equal(np.array([t[0] for t in got[i]], np.float32),
                                      np.array([t[0] for t in want], np.float32))
    assert bs.launches < sum(len(w) for w in got)  # batched: fewer launches than distances

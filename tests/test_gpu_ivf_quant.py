"""IVF-SQ8 and IVF-PQ on the GPU against the oracle's composition (IVF
probing + SQ8 scores / PQ ADC sums, stable candidate order).  Probing is
exact and the scores are exact integers or fixed-order fp32 sums, so
scores, distances and ids must be bit-identical."""
import numpy as np
import pytest

from oracle import oracle as O
from vectorstorekit_amd import (IVFConfiguration, IVFIndex, ProductQuantizer, ScalarQuantizer,
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
    idx.insert(x)
    return idx


# (nlist, n, d, nq, nprobe, k, per_dim)
SQ_SHAPES = [(64, 20_000, 128, 100, 8, 10, True), (37, 5000, 33, 50, 5, 7, False),
             (16, 3000, 24, 40, 16, 20, True), (8, 600, 200, 17, 2, 300, True)]


@pytest.mark.parametrize("shape", SQ_SHAPES)
def test_ivf_sq8_bit_exact(ctx, shape):
    nlist, n, d, nq, nprobe, k, per_dim = shape
    x, q, c = _mixture(nlist + d, nlist, n, d, nq)
    idx = _index(ctx, c, x, nprobe)
    sq = ScalarQuantizer(ctx, per_dim=per_dim)
    sq.train(x)
    idx.encodeSQ8(sq)
    score, ids = idx.searchSQ8(q, k)
    codes = O.sq8_encode(x, sq.scale, sq.offset)
    qc = O.sq8_encode(q, sq.scale, sq.offset)
    es, ei = O.ivf_sq8_search(q, qc, codes, np.arange(n), O.ivf_assign(x, c), c, nprobe, k)
    np.testing.assert_array_equal(score, es)
    np.testing.assert_array_equal(ids, ei)


# (nlist, n, M, dsub, nq, nprobe, k)
PQ_SHAPES = [(64, 20_000, 16, 8, 100, 8, 10), (37, 5000, 8, 4, 50, 5, 7),
             (16, 3000, 6, 5, 40, 16, 20), (8, 600, 16, 12, 17, 2, 300)]


@pytest.mark.parametrize("shape", PQ_SHAPES)
def test_ivf_pq_bit_exact(ctx, shape):
    nlist, n, M, dsub, nq, nprobe, k = shape
    d = M * dsub
    x, q, c = _mixture(nlist + M, nlist, n, d, nq)
    rng = np.random.default_rng(M)
    cb = x[rng.choice(n, 256, replace=False)].reshape(256, M, dsub).transpose(1, 0, 2).copy()
    idx = _index(ctx, c, x, nprobe)
    pq = ProductQuantizer(ctx, cb)
    idx.encodePQ(pq)
    dist, ids = idx.searchPQ(q, k)
    codes = O.pq_encode(x, cb)
    ed, ei = O.ivf_pq_search(q, cb, codes, np.arange(n), O.ivf_assign(x, c), c, nprobe, k)
    np.testing.assert_array_equal(dist, ed)
    np.testing.assert_array_equal(ids, ei)


def test_ivf_sq8_all_lists_is_the_flat_sq8_scan(ctx):
    x, q, c = _mixture(5, 16, 4000, 64, 30)
    idx = _index(ctx, c, x, 16)
    sq = ScalarQuantizer(ctx)
    sq.train(x)
    idx.encodeSQ8(sq)
    score, _ = idx.searchSQ8(q, 25, strategy="exact")
    codes = O.sq8_encode(x, sq.scale, sq.offset)
    es, _ = O.sq8_search(O.sq8_encode(q, sq.scale, sq.offset), codes, 25)
    np.testing.assert_array_equal(score, es)


def test_ivf_codes_follow_inserts(ctx):
    x, q, c = _mixture(9, 8, 2000, 32, 10)
    idx = _index(ctx, c, x[:1500], 3)
    sq = ScalarQuantizer(ctx)
    sq.train(x)
    with pytest.raises(VSKError):
        idx.searchSQ8(q, 5)  # nothing encoded yet
    idx.encodeSQ8(sq)
    idx.insert(x[1500:])
    with pytest.raises(VSKError):
        idx.searchSQ8(q, 5)  # stale codes
    idx.encodeSQ8(sq)
    score, ids = idx.searchSQ8(q, 5)
    codes = O.sq8_encode(x, sq.scale, sq.offset)
    es, ei = O.ivf_sq8_search(q, O.sq8_encode(q, sq.scale, sq.offset), codes, np.arange(2000),
                              O.ivf_assign(x, c), c, 3, 5)
    np.testing.assert_array_equal(score, es)
    np.testing.assert_array_equal(ids, ei)
    with pytest.raises(VSKError):
        idx.searchPQ(q, 5)  # the index holds SQ8 codes


def test_ivf_index_file_round_trip(ctx, tmp_path):
    x, q, c = _mixture(21, 32, 6000, 40, 25)
    idx = _index(ctx, c, x[:5000], 6)
    idx.insert(x[5000:], ids=np.arange(5000, 6000, dtype=np.int64) * 7)
    sq = ScalarQuantizer(ctx)
    sq.train(x)
    idx.encodeSQ8(sq)
    path = str(tmp_path / "ivf.vsk")
    idx.save(path)
    back = IVFIndex.load(ctx, path, sq8=sq)
    assert back.configuration.numberOfProbes == 6  # the configuration travels in the file
    np.testing.assert_array_equal(back.getCentroids(), c)
    # the SQ8 parameters travel too: without a quantizer the loaded index
    # searches its codes with the stored one; a different one is refused
    alone = IVFIndex.load(ctx, path)
    for a, b in zip(idx.searchSQ8(q, 9), alone.searchSQ8(q, 9)):
        np.testing.assert_array_equal(a, b)
    other = ScalarQuantizer(ctx)
    other.train(x[:100])
    with pytest.raises(VSKError) as e:
        IVFIndex.load(ctx, path, sq8=other)
    assert e.value.status == -4
    np.testing.assert_array_equal(back.list_sizes(), idx.list_sizes())
    for a, b in zip(idx.search(q, 9), back.search(q, 9)):
        np.testing.assert_array_equal(a, b)
    for a, b in zip(idx.searchSQ8(q, 9), back.searchSQ8(q, 9)):
        np.testing.assert_array_equal(a, b)
    # later inserts take the next ids in both
    idx.insert(x[:10])
    back.insert(x[:10])
    for a, b in zip(idx.search(q, 9), back.search(q, 9)):
        np.testing.assert_array_equal(a, b)
    # stale codes are not written
    idx.save(path)
    with pytest.raises(VSKError):
        IVFIndex.load(ctx, path, sq8=sq).searchSQ8(q, 3)


def test_ivf_index_file_pq_round_trip(ctx, tmp_path):
    x, q, c = _mixture(22, 16, 3000, 32, 20)
    rng = np.random.default_rng(1)
    cb = x[rng.choice(3000, 256, replace=False)].reshape(256, 8, 4).transpose(1, 0, 2).copy()
    idx = _index(ctx, c, x, 4)
    pq = ProductQuantizer(ctx, cb)
    idx.encodePQ(pq)
    path = str(tmp_path / "ivfpq.vsk")
    idx.save(path)
    back = IVFIndex.load(ctx, path, pq=pq)
    for a, b in zip(idx.searchPQ(q, 11), back.searchPQ(q, 11)):
        np.testing.assert_array_equal(a, b)
    # a quantizer of the same shape with other codebooks is refused
    cb2 = cb.copy()
    cb2[3, 17, 1] += 1.0
    with pytest.raises(VSKError) as e:
        IVFIndex.load(ctx, path, pq=ProductQuantizer(ctx, cb2)).searchPQ(q, 11)
    assert e.value.status == -4


def _fnv1a(b: bytes) -> int:
    h = 0xcbf29ce484222325
    for byte in b:
        h = ((h ^ byte) * 0x100000001b3) & 0xFFFFFFFFFFFFFFFF
    return h


def test_ivf_index_file_crafted_headers_and_codes(ctx, tmp_path):
    """Files with a valid checksum but bad contents are refused: a header
    whose sizes overflow, and a PQ code past the codebook size."""
    import struct

    x, q, c = _mixture(24, 8, 600, 16, 4)
    rng = np.random.default_rng(2)
    cb = x[rng.choice(600, 16, replace=False)].reshape(16, 4, 4).transpose(1, 0, 2).copy()
    idx = _index(ctx, c, x, 2)
    pq = ProductQuantizer(ctx, cb)  # ksub = 16
    idx.encodePQ(pq)
    path = tmp_path / "ivfpq.vsk"
    idx.save(str(path))
    raw = path.read_bytes()

    def seal(body: bytes) -> bytes:
        return body + struct.pack("<Q", _fnv1a(body))

    assert seal(raw[:-8]) == raw
    nlist, d = struct.unpack_from("<ii", raw, 8)
    total = struct.unpack_from("<q", raw, 16)[0]
    stride = struct.unpack_from("<i", raw, 36)[0]
    codes_at = 64 + 4 * nlist * d + 8 * (nlist + 1) + 8 * total + 4 * total * d
    assert raw[codes_at] < 16
    bad_code = bytearray(raw[:-8])
    bad_code[codes_at + stride * 5 + 1] = 200  # row 5, segment 1: >= ksub
    cases = {"code past ksub": seal(bytes(bad_code))}
    for name, dd, nn in (("huge d", 0x7FFFFFFF, nlist), ("huge nlist", d, 0x7FFFFFFF),
                         ("negative d", -4, nlist)):
        b = bytearray(raw[:-8])
        struct.pack_into("<ii", b, 8, nn, dd)
        cases[name] = seal(bytes(b))
    b = bytearray(raw[:-8])
    struct.pack_into("<q", b, 56, 1 << 40)  # metadata size
    cases["huge meta"] = seal(bytes(b))
    for name, blob in cases.items():
        bad = tmp_path / "bad.vsk"
        bad.write_bytes(blob)
        with pytest.raises(VSKError) as e:
            IVFIndex.load(ctx, str(bad), pq=pq)
        assert e.value.status == -10, name


def test_ivf_index_file_damage(ctx, tmp_path):
    x, q, c = _mixture(23, 8, 800, 16, 5)
    idx = _index(ctx, c, x, 2)
    path = tmp_path / "ivf.vsk"
    idx.save(str(path))
    raw = path.read_bytes()
    cases = {"flipped": raw[:3000] + bytes([raw[3000] ^ 1]) + raw[3001:],
             "truncated": raw[:-9], "magic": b"VSKIVF01" + raw[8:], "longer": raw + b"\0"}
    for name, blob in cases.items():
        bad = tmp_path / f"{name}.vsk"
        bad.write_bytes(blob)
        with pytest.raises(VSKError) as e:
            IVFIndex.load(ctx, str(bad))
        assert e.value.status == -10, name
    with pytest.raises(VSKError):
        IVFIndex.load(ctx, str(tmp_path / "missing.vsk"))


@pytest.mark.parametrize("kind", ["sq8", "pq"])
def test_ivf_codes_only(ctx, tmp_path, kind):
    """vsk_ivf_drop_rows: the index keeps its codes and frees its fp32 rows.
    Searches answer exactly as before (and as the oracle); the index's
    device memory shrinks by the rows; inserts after it are encoded with the
    stored quantizer and rank as the oracle over all rows; removes keep the
    remaining codes; the codes-only file has no rows section and loads back
    to the same answers; the calls that need rows raise."""
    nlist, n, d, nq, nprobe, k = 32, 12_000, 64, 60, 6, 20
    x, q, c = _mixture(77 if kind == "sq8" else 78, nlist, n, d, nq)
    idx = _index(ctx, c, x[:10_000], nprobe)
    if kind == "sq8":
        sq = ScalarQuantizer(ctx, per_dim=True)
        sq.train(x)
        idx.encodeSQ8(sq)
        run = lambda ix: ix.searchSQ8(q, k)
        codes = O.sq8_encode(x, sq.scale, sq.offset)
        qc = O.sq8_encode(q, sq.scale, sq.offset)
        want = lambda keep: O.ivf_sq8_search(q, qc, codes[keep], keep, O.ivf_assign(x[keep], c),
                                             c, nprobe, k)
    else:
        rng = np.random.default_rng(3)
        cb = x[rng.choice(n, 256, replace=False)].reshape(256, 16, 4).transpose(1, 0, 2).copy()
        pq = ProductQuantizer(ctx, cb)
        idx.encodePQ(pq)
        run = lambda ix: ix.searchPQ(q, k)
        codes = O.pq_encode(x, cb)
        want = lambda keep: O.ivf_pq_search(q, cb, codes[keep], keep, O.ivf_assign(x[keep], c),
                                            c, nprobe, k)
    s0, i0 = run(idx)
    co, before = idx.storage()
    assert not co
    idx.dropRows()
    co, after = idx.storage()
    assert co and idx.codesOnly
    assert before - after >= 10_000 * d * 4  # the rows (and any plane) are gone
    s1, i1 = run(idx)
    np.testing.assert_array_equal(s1, s0)
    np.testing.assert_array_equal(i1, i0)
    with pytest.raises(VSKError):
        idx.search(q, k)
    with pytest.raises(VSKError):
        if kind == "sq8":
            idx.encodeSQ8(sq)
        else:
            idx.encodePQ(pq)
    # inserts are encoded with the stored quantizer
    idx.insert(x[10_000:])
    s2, i2 = run(idx)
    es, ei = want(np.arange(n))
    np.testing.assert_array_equal(s2, es)
    np.testing.assert_array_equal(i2, ei)
    # removes keep the other rows' codes
    gone = np.arange(0, n, 3)
    assert idx.remove(gone) == gone.size
    keep = np.setdiff1d(np.arange(n), gone)
    s3, i3 = run(idx)
    es, ei = want(keep)
    np.testing.assert_array_equal(s3, es)
    np.testing.assert_array_equal(i3, ei)
    # the file has no rows section and answers the same after loading
    path = str(tmp_path / f"codes_only_{kind}.ivf")
    idx.save(path)
    import os

    assert os.path.getsize(path) < keep.size * d * 4  # smaller than the rows alone
    back = IVFIndex.load(ctx, path, pq=None if kind == "sq8" else pq)
    assert back.codesOnly
    s4, i4 = run(back)
    np.testing.assert_array_equal(s4, s3)
    np.testing.assert_array_equal(i4, i3)

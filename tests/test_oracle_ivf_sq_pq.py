"""Pins the oracle's IVF, int8-SQ and PQ functions.

Each check is chosen so a plausible slip in the oracle fails it: IVF with
every list probed must equal flat search; the reference's own IVF and SQ
known answers; integer scores against int64 brute force; SQ codes against
numpy's fp32 arithmetic; PQ tables against float64 and against an explicit
fp32 left fold; the ADC identity ADC(q, code) = |q - decode(code)|^2.
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


def _lex(D, k):
    idx = np.lexsort((np.broadcast_to(np.arange(D.shape[1]), D.shape), D), axis=1)[:, :k]
    return np.take_along_axis(D, idx, 1), idx


# ---------------------------------------------------------------- IVF ---

def _mixture(seed, ncent, n, d, nq):
    rng = np.random.default_rng(seed)
    cent = (2.0 * rng.standard_normal((ncent, d))).astype(np.float32)
    a = rng.integers(0, ncent, n)
    x = (cent[a] + 0.5 * rng.standard_normal((n, d))).astype(np.float32)
    qa = rng.integers(0, ncent, nq)
    q = (cent[qa] + 0.5 * rng.standard_normal((nq, d))).astype(np.float32)
    c = (cent + 0.1 * rng.standard_normal(cent.shape)).astype(np.float32)
    return x, q, c


def test_ivf_assign_is_first_argmin():
    x, q, c = _mixture(0, 32, 2000, 16, 5)
    got = O.ivf_assign(x, c)
    D = np.sqrt(O.distances(x, c, O.L2SQ))
    np.testing.assert_array_equal(got, np.argmin(D, axis=1))  # argmin = first min
    # duplicate centroid: the first copy wins
    c2 = np.concatenate([c, c[:1]])
    assert (O.ivf_assign(x, c2) != 32).all()


def test_ivf_probe_is_stable_sort():
    x, q, c = _mixture(1, 64, 10, 16, 20)
    c[5] = c[9]  # tie: index 5 before 9
    got = O.ivf_probe(q, c, 8)
    D = np.sqrt(O.distances(q, c, O.L2SQ))
    np.testing.assert_array_equal(got, _lex(D, 8)[1])


def test_ivf_all_lists_equals_flat():
    x, q, c = _mixture(2, 16, 3000, 24, 30)
    lists = O.ivf_assign(x, c)
    ids = np.arange(len(x), dtype=np.int64) + 1000
    d, i = O.ivf_search(q, x, ids, lists, c, 16, 10)
    fd, fi = O.search_flat(q, x, 10, O.L2)
    np.testing.assert_array_equal(d, fd)
    # same set; order may differ only between exactly equal distances
    for a, b in zip(i, fi + 1000):
        assert set(a) == set(b)


def test_ivf_squared_all_lists_equals_flat_l2sq():
    """The squared variant ranks on the sum itself: probing every list gives
    flat L2SQ's distances exactly, and its sqrt is the default output."""
    x, q, c = _mixture(4, 16, 3000, 24, 30)
    lists = O.ivf_assign(x, c)
    ids = np.arange(len(x), dtype=np.int64)
    d2, i2 = O.ivf_search(q, x, ids, lists, c, 16, 10, squared=True)
    fd, fi = O.search_flat(q, x, 10, O.L2SQ)
    np.testing.assert_array_equal(d2, fd)
    for a, b in zip(i2, fi):
        assert set(a) == set(b)
    d1, _ = O.ivf_search(q, x, ids, lists, c, 16, 10)
    np.testing.assert_array_equal(d1, np.sqrt(d2))


def test_ivf_candidates_in_probe_order():
    x, q, c = _mixture(3, 8, 500, 8, 10)
    lists = O.ivf_assign(x, c)
    ids = np.arange(len(x), dtype=np.int64)
    probes = O.ivf_probe(q, c, 3)
    d, i = O.ivf_search(q, x, ids, lists, c, 3, 20)
    for qi in range(len(q)):
        cand = np.concatenate([np.nonzero(lists == l)[0] for l in probes[qi]])
        dist = np.sqrt(O.distances(q[qi:qi + 1], x[cand], O.L2SQ))[0]
        order = np.lexsort((np.arange(len(cand)), dist))[:20]
        np.testing.assert_array_equal(i[qi], cand[order])
        np.testing.assert_array_equal(d[qi], dist[order])


def test_ivf_reference_basic_kat():
    # IVFIndexTests.swift:160-201
    k = kats()["ivf_basic"]
    c = np.array(k["training"][:4], np.float32)  # the 4 basis vectors as centroids
    x = np.array([k["inserted"]], np.float32)
    lists = O.ivf_assign(x, c)
    d, i = O.ivf_search(np.array([k["query"]], np.float32), x, np.array([1], np.int64),
                        lists, c, k["nprobe"], 1)
    assert i[0, 0] == 1  # "vec1"


def test_ivf_reference_exact_self_kat():
    # IVFIndexTests.swift:203-260: .exact search of an inserted row finds it
    k = kats()["ivf_exact_self"]
    rng = np.random.default_rng(4)
    centers = rng.standard_normal((k["clusters"], k["dim"])).astype(np.float32)
    data = (np.repeat(centers, k["per_cluster"], 0) +
            0.1 * rng.standard_normal((k["clusters"] * k["per_cluster"], k["dim"]))).astype(np.float32)
    c = O.kmeans(data, k["clusters"], iters=5, seed=1)
    x = data[:k["inserted"]]
    lists = O.ivf_assign(x, c)
    d, i = O.ivf_search(data[k["query_row"]:k["query_row"] + 1], x,
                        np.arange(len(x), dtype=np.int64), lists, c, k["clusters"], k["k"])
    assert i[0, 0] == k["query_row"] and d[0, 0] == 0.0


# ----------------------------------------------------------------- SQ ---

def test_sq8_params_and_codes_match_numpy_fp32():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((300, 17)).astype(np.float32)
    for per_dim in (True, False):
        s, o = O.sq8_train(x, per_dim)
        mn = x.min(0) if per_dim else np.array([x.min()])
        mx = x.max(0) if per_dim else np.array([x.max()])
        es = (np.float32(255.0) / (mx - mn).astype(np.float32)).astype(np.float32)
        eo = ((-mn.astype(np.float32)) * es - np.float32(128.0)).astype(np.float32)
        np.testing.assert_array_equal(s, es)
        np.testing.assert_array_equal(o, eo)
        codes = O.sq8_encode(x, s, o)
        t = (x * s).astype(np.float32) + o  # two fp32 roundings, as vDSP_vsmsa
        want = np.clip(np.trunc(t), -128, 127).astype(np.int8)
        np.testing.assert_array_equal(codes, want)
        # round trip within one quantization step
        back = O.sq8_decode(codes, s, o)
        step = (mx - mn) / 255.0
        assert (np.abs(back - x) <= step * 1.0001 + 1e-6).all()


def test_sq8_reference_roundtrip_kat():
    # ScalarQuantizerTests.swift:55-74
    k = kats()["sq8_roundtrip"]
    v = np.array([k["vector"]], np.float32)
    s, o = O.sq8_train(v, per_dim=False)
    back = O.sq8_decode(O.sq8_encode(v, s, o), s, o)
    assert np.abs(back - v).max() <= k["tolerance"]


def test_sq8_search_is_integer_brute_force():
    rng = np.random.default_rng(6)
    codes = rng.integers(-128, 128, (2000, 40)).astype(np.int8)
    qc = rng.integers(-128, 128, (9, 40)).astype(np.int8)
    codes[100] = codes[50]  # tie: id 50 first
    qc[0] = codes[50]
    sc, ids = O.sq8_search(qc, codes, 25)
    S = qc.astype(np.int64) @ codes.astype(np.int64).T
    want_d, want_i = _lex(-S, 25)
    np.testing.assert_array_equal(ids, want_i)
    np.testing.assert_array_equal(sc, -want_d)
    assert ids[0, 0] == 50 and ids[0, 1] == 100


# ----------------------------------------------------------------- PQ ---

def _pq_setup(seed=7, n=3000, M=4, ksub=16, dsub=4, nq=6):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, M * dsub)).astype(np.float32)
    cb = np.stack([O.kmeans(x[:, m * dsub:(m + 1) * dsub].copy(), ksub, iters=4, seed=m)
                   for m in range(M)])
    q = rng.standard_normal((nq, M * dsub)).astype(np.float32)
    return x, cb, q


def test_pq_lut_values():
    x, cb, q = _pq_setup()
    M, ksub, dsub = cb.shape
    lut = O.pq_lut(q[0], cb)
    want = ((q[0].reshape(M, 1, dsub).astype(np.float64) - cb) ** 2).sum(-1)
    np.testing.assert_allclose(lut, want, rtol=1e-6, atol=1e-7)
    # exact fp32 left fold over the segment, no FMA
    for m, c in [(0, 0), (1, 5), (3, 15)]:
        s = np.float32(0)
        for j in range(dsub):
            t = np.float32(q[0, m * dsub + j] - cb[m, c, j])
            s = np.float32(s + np.float32(t * t))
        assert lut[m, c] == s
    # a query segment equal to a codeword gives a zero entry
    qq = q[0].copy()
    qq[dsub:2 * dsub] = cb[1, 7]
    assert O.pq_lut(qq, cb)[1, 7] == 0.0


def test_pq_encode_is_argmin():
    x, cb, q = _pq_setup()
    M, ksub, dsub = cb.shape
    codes = O.pq_encode(x, cb)
    for m in range(M):
        seg = x[:, m * dsub:(m + 1) * dsub]
        D = O.distances(seg, cb[m], O.L2SQ)
        np.testing.assert_array_equal(codes[:, m], np.argmin(D, 1))


def test_pq_adc_identity():
    # ADC(q, code) = |q - decode(code)|^2 (ProductQuantizer.swift:187-206, 341-356)
    x, cb, q = _pq_setup()
    codes = O.pq_encode(x, cb)
    dec = O.pq_decode(codes, cb)
    for qi in range(len(q)):
        adc = O.pq_adc_scan(O.pq_lut(q[qi], cb), codes)
        want = ((q[qi].astype(np.float64) - dec) ** 2).sum(1)
        np.testing.assert_allclose(adc, want, rtol=1e-5, atol=1e-5)
    # the sum is formed m-ascending in fp32
    lut = O.pq_lut(q[0], cb)
    s = np.float32(0)
    for m in range(cb.shape[0]):
        s = np.float32(s + lut[m, codes[0, m]])
    assert O.pq_adc_scan(lut, codes[:1])[0] == s


def test_pq_search_brute_force_and_rerank():
    x, cb, q = _pq_setup()
    codes = O.pq_encode(x, cb)
    d, i = O.pq_search(q, cb, codes, 50, 50)
    for qi in range(len(q)):
        adc = O.pq_adc_scan(O.pq_lut(q[qi], cb), codes)
        wd, wi = _lex(adc[None], 50)
        np.testing.assert_array_equal(i[qi], wi[0])
        np.testing.assert_array_equal(d[qi], np.sqrt(wd[0]).astype(np.float32))
    rd, ri = O.pq_search(q, cb, codes, 50, 10, x=x, rerank_metric=O.L1)
    for qi in range(len(q)):
        cand = i[qi]
        l1 = O.distances(q[qi:qi + 1], x[cand], O.L1)[0]
        order = np.lexsort((cand, l1))[:10]
        np.testing.assert_array_equal(ri[qi], cand[order])
        np.testing.assert_array_equal(rd[qi], l1[order])


def test_decoders_exact():
    """dequantizeFromInt8 (ScalarQuantizer.swift:568-580) is numpy's fp32
    (code - offset) / scale; PQ decode (ProductQuantizer.swift:142-160) is
    numpy indexing of each segment's codebook."""
    rng = np.random.default_rng(9)
    codes = rng.integers(-128, 128, (300, 17)).astype(np.int8)
    s = rng.random(17).astype(np.float32) * 50 + 1
    o = (rng.standard_normal(17) * 30).astype(np.float32)
    want = (codes.astype(np.float32) - o) / s
    np.testing.assert_array_equal(O.sq8_decode(codes, s, o), want.astype(np.float32))
    cb = rng.standard_normal((4, 256, 5)).astype(np.float32)
    pc = rng.integers(0, 256, (200, 4)).astype(np.uint8)
    want = np.concatenate([cb[m][pc[:, m]] for m in range(4)], axis=1)
    np.testing.assert_array_equal(O.pq_decode(pc, cb), want)


def test_ivf_coded_oracles_over_every_list():
    """nprobe = nlist: the IVF-SQ8 / IVF-PQ oracles see every row, so their
    scores and distances are those of the flat SQ8 scan and of the
    non-re-ranked PQ search; and a hand-built candidate set for one query
    (the numpy-float64-nearest lists) gives the same top scores."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal((900, 16)).astype(np.float32)
    q = rng.standard_normal((6, 16)).astype(np.float32)
    c = rng.standard_normal((12, 16)).astype(np.float32)
    lo = O.ivf_assign(x, c)
    s, o = O.sq8_train(x)
    codes, qc = O.sq8_encode(x, s, o), O.sq8_encode(q, s, o)
    es, _ = O.ivf_sq8_search(q, qc, codes, np.arange(900), lo, c, 12, 40)
    fs, _ = O.sq8_search(qc, codes, 40)
    np.testing.assert_array_equal(es, fs)
    cb = x[:256 * 1].reshape(256, 4, 4).transpose(1, 0, 2).copy()
    pc = O.pq_encode(x, cb)
    ed, _ = O.ivf_pq_search(q, cb, pc, np.arange(900), lo, c, 12, 40)
    fd, _ = O.pq_search(q, cb, pc, 40, 40)
    np.testing.assert_array_equal(ed, fd)
    # three probes of query 0 by float64 distance
    d0 = ((c.astype(np.float64) - q[0]) ** 2).sum(1)
    rows = np.nonzero(np.isin(lo, np.argsort(d0)[:3]))[0]
    sc = codes[rows].astype(np.int64) @ qc[0].astype(np.int64)
    ps, _ = O.ivf_sq8_search(q[:1], qc[:1], codes, np.arange(900), lo, c, 3, 10)
    np.testing.assert_array_equal(ps[0], np.sort(sc)[::-1][:10])


def test_sq8_search_scores_past_float_precision():
    """Scores above 2^24 that differ by 1: a float key would merge them and
    fall back to the row order; the int64 keys keep the higher score first.
    Pinned by int64 brute force."""
    d = 2048
    q = np.full((1, d), 127, np.int8)
    q[0, 5] = 1
    codes = np.full((4, d), 127, np.int8)
    codes[0, 5] = 126  # score S + 126 at row 0
    codes[2, 7] = 126  # score S + 127 - 127 at row 2
    score, ids = O.sq8_search(q, codes, 4)
    ref = codes.astype(np.int64) @ q[0].astype(np.int64)
    order = np.lexsort((np.arange(4), -ref))
    assert ref[1] - ref[0] == 1 and ref[0] > 2 ** 24
    np.testing.assert_array_equal(ids[0], order)
    np.testing.assert_array_equal(score[0], ref[order])

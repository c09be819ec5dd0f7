"""The oracle's matrixMultiply (vsko_matmul): each entry summed over the
inner dimension in order from 0, a product and then a sum, as the
reference's CPU loop (Acceleration/Metal/MetalMatrixCompute.swift:791-806).

Pinned by the reference's own known answer (MetalComponentTests.swift:
244-271, fixture tests/golden/reference_kats.json), by an explicit numpy fp32
left fold on random matrices (bit for bit; a pairwise or fused sum changes
some entries, which the same check would catch), by float64 within
tolerance, and by the identity matrix."""
import json
import os

import numpy as np

from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))


def test_reference_known_answer():
    k = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))["matrix_multiply"]
    c = O.matmul(np.array(k["a"], np.float32), np.array(k["b"], np.float32))
    np.testing.assert_array_equal(c, np.array(k["c"], np.float32))


def _fold(a, b):
    m, kk = a.shape
    n = b.shape[1]
    out = np.empty((m, n), np.float32)
    for i in range(m):
        for j in range(n):
            s = np.float32(0.0)
            for t in range(kk):
                s = np.float32(s + np.float32(a[i, t] * b[t, j]))
            out[i, j] = s
    return out


def test_left_fold_bit_exact():
    rng = np.random.default_rng(5)
    for m, kk, n in ((7, 13, 5), (3, 64, 9), (1, 1, 1), (4, 129, 2)):
        a = rng.standard_normal((m, kk)).astype(np.float32)
        b = rng.standard_normal((kk, n)).astype(np.float32)
        np.testing.assert_array_equal(O.matmul(a, b).view(np.uint32), _fold(a, b).view(np.uint32))


def test_order_matters_and_float64():
    rng = np.random.default_rng(6)
    a = rng.standard_normal((40, 300)).astype(np.float32)
    b = rng.standard_normal((300, 30)).astype(np.float32)
    c = O.matmul(a, b)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    np.testing.assert_allclose(c, ref, rtol=1e-4, atol=1e-4)
    # a fused multiply-add per step (one rounding instead of two) gives
    # other bits in some entries: the fold above pins the unfused order
    fused = np.empty_like(c)
    for i in range(a.shape[0]):
        for j in range(b.shape[1]):
            s = 0.0
            for t in range(a.shape[1]):
                s = float(np.float32(s + float(a[i, t]) * float(b[t, j])))
            fused[i, j] = s
    assert (fused != c).any()


def test_identity():
    rng = np.random.default_rng(7)
    a = rng.standard_normal((11, 17)).astype(np.float32)
    np.testing.assert_array_equal(O.matmul(a, np.eye(17, dtype=np.float32)), a)

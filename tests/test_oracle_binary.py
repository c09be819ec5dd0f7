"""Pins the oracle's binary quantization and Hamming search
(oracle/vsk_oracle.c: vsko_binary_encode, vsko_bin_hamming, vsko_bin_search,
VSKO_HAMMING) against numpy's bit routines and brute force.

Reference: AccelerateOptimizer.binaryQuantize
(Acceleration/AccelerateOptimizer.swift:447-481), binaryHammingDistance
(Acceleration/Metal/Shaders/QuantizationShaders.metal:285-305) and the float
hammingDistance (Core/Distance/UnifiedDistanceComputation.swift:249-261)."""
import numpy as np

from oracle import oracle as O


def test_encode_is_little_endian_packbits():
    """bit i = x_i > 0 in byte i/8 at bit i%8: numpy's packbits with
    bitorder='little' of (x > 0); zeros, negatives and NaN give 0."""
    rng = np.random.default_rng(1)
    for d in [1, 7, 8, 9, 37, 128, 1000]:
        x = rng.standard_normal((50, d)).astype(np.float32)
        x[0, :] = 0.0
        x[1, ::3] = np.nan
        x[2, ::2] = -0.0
        np.testing.assert_array_equal(O.binary_encode(x),
                                      np.packbits(x > 0, axis=1, bitorder="little"))


def test_hamming_two_reference_definitions_agree():
    """popcount(a xor b) of the codes equals the reference's float
    hammingDistance (count of unequal components) on the unpacked 0/1
    vectors, and numpy's unpackbits count."""
    rng = np.random.default_rng(2)
    d = 77
    a = np.packbits(rng.random((20, d)) > 0.5, axis=1, bitorder="little")
    b = np.packbits(rng.random((30, d)) > 0.5, axis=1, bitorder="little")
    ua = np.unpackbits(a, axis=1, bitorder="little")[:, :d].astype(np.float32)
    ub = np.unpackbits(b, axis=1, bitorder="little")[:, :d].astype(np.float32)
    fl = O.distances(ua, ub, O.HAMMING)
    for i in range(20):
        for j in range(30):
            h = int(np.unpackbits(a[i] ^ b[j]).sum())
            assert O.lib().vsko_bin_hamming(a[i].ctypes.data, b[j].ctypes.data, a.shape[1]) == h
            assert fl[i, j] == h


def test_float_hamming_counts_unequal_components():
    rng = np.random.default_rng(3)
    q = rng.integers(0, 3, (6, 40)).astype(np.float32)
    x = rng.integers(0, 3, (90, 40)).astype(np.float32)
    q[0, 5] = np.nan  # NaN differs from everything, itself included
    x[:, 5][:3] = np.nan
    ref = (q[:, None, :] != x[None, :, :]).sum(-1).astype(np.float32)
    np.testing.assert_array_equal(O.distances(q, x, O.HAMMING), ref)


def test_bin_search_brute_force_with_ties():
    """(distance, id) order against lexsort; short integer distances make
    large ties at the k-th distance; k > n pads with (INT32_MAX, -1)."""
    rng = np.random.default_rng(4)
    d = 24
    x = np.packbits(rng.random((3000, d)) > 0.5, axis=1, bitorder="little")
    q = np.packbits(rng.random((25, d)) > 0.5, axis=1, bitorder="little")
    ux = np.unpackbits(x, axis=1, bitorder="little")[:, :d]
    uq = np.unpackbits(q, axis=1, bitorder="little")[:, :d]
    full = (uq[:, None, :] != ux[None, :, :]).sum(-1)
    od, oi = O.bin_search(q, x, d, 50)
    for i in range(25):
        order = np.lexsort((np.arange(3000), full[i]))[:50]
        np.testing.assert_array_equal(oi[i], order)
        np.testing.assert_array_equal(od[i], full[i][order])
    od, oi = O.bin_search(q[:2], x[:5], d, 8)
    assert (oi[:, 5:] == -1).all() and (od[:, 5:] == 0x7FFFFFFF).all()

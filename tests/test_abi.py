"""The C-ABI library: it loads without a GPU, exports every function that
include/vsk_hip.h declares, and the Python binding table matches the header.
No compute calls (this runs on CPU-only machines)."""
import ctypes
import os
import re

import numpy as np
import pytest

import vectorstorekit_amd as vsk
from vectorstorekit_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vsk_hip.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vsk_[a-z0-9_]+)\s*\(", text)))


def test_library_loads():
    assert os.path.exists(_lib.library_path()), "run __graft_entry__.build() first"
    lib = vsk.load_library()
    assert isinstance(lib, ctypes.CDLL)


def test_every_declared_symbol_is_exported():
    lib = vsk.load_library()
    declared = header_functions()
    assert len(declared) >= 30
    missing = [f for f in declared if not hasattr(lib, f)]
    assert missing == []


def test_binding_table_matches_header():
    assert sorted(_lib.SIGNATURES) == header_functions()


def test_constants_match_header():
    text = open(HEADER).read()
    defs = dict(re.findall(r"#define (VSK_\w+) \(?(-?\d+)\)?", text))
    assert int(defs["VSK_METRIC_L2SQ"]) == _lib.METRIC_L2SQ
    assert int(defs["VSK_METRIC_L2"]) == _lib.METRIC_L2
    assert int(defs["VSK_METRIC_COSINE"]) == _lib.METRIC_COSINE
    assert int(defs["VSK_METRIC_COSINE_NORMALIZED"]) == _lib.METRIC_COSINE_NORMALIZED
    assert int(defs["VSK_METRIC_DOT"]) == _lib.METRIC_DOT
    assert int(defs["VSK_METRIC_L1"]) == _lib.METRIC_L1
    assert int(defs["VSK_MAX_K"]) == _lib.MAX_K
    for code, name in _lib.STATUS_NAMES.items():
        assert code in [int(v) for k, v in defs.items() if k.startswith("VSK_ERR_")]


def test_oracle_metric_codes_match():
    from oracle import oracle as O

    assert (O.L2SQ, O.L2, O.COSINE, O.COSINE_NORMALIZED, O.DOT, O.L1) == (
        _lib.METRIC_L2SQ, _lib.METRIC_L2, _lib.METRIC_COSINE,
        _lib.METRIC_COSINE_NORMALIZED, _lib.METRIC_DOT, _lib.METRIC_L1)


def test_null_and_no_device_errors():
    """Host-side argument checks that need no device; on a machine without
    a GPU vsk_create reports deviceNotAvailable."""
    lib = vsk.load_library()
    assert lib.vsk_create(0, None) == -2
    assert lib.vsk_destroy(None) == 0
    assert lib.vsk_last_error(None) == b"null context"
    assert lib.vsk_db_info(None, None, None) == -2
    import torch

    if not torch.cuda.is_available():
        h = ctypes.c_void_p()
        assert lib.vsk_create(0, ctypes.byref(h)) == -1
        with pytest.raises(vsk.VSKError) as e:
            vsk.Context(0)
        assert e.value.kind == "deviceNotAvailable"


def test_product_does_not_import_oracle():
    """The shipped package never reaches into oracle/ (the checker)."""
    pkg = os.path.join(ROOT, "vectorstorekit_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".hpp", ".h", ".cpp")) or f == "Makefile":
                text = open(os.path.join(dirpath, f), errors="ignore").read()
                assert "from oracle" not in text and "import oracle" not in text, f
                assert "libvsk_oracle" not in text, f


def test_row_bitmap_layout():
    """The row filter the C ABI takes: bit i % 32 of word i // 32; from a
    boolean mask or from allowed indices, padded with zero words."""
    mask = np.zeros(70, np.bool_)
    mask[[0, 5, 31, 32, 69]] = True
    bm = _lib.row_bitmap(mask)
    assert bm.dtype == np.uint32 and bm.size == 3
    assert list(bm) == [(1 << 0) | (1 << 5) | (1 << 31), 1, 1 << 5]
    np.testing.assert_array_equal(_lib.row_bitmap([0, 5, 31, 32, 69]), bm)
    np.testing.assert_array_equal(_lib.row_bitmap(np.array([], np.int64), 64),
                                  np.zeros(2, np.uint32))
    unpacked = np.unpackbits(bm.view(np.uint8), bitorder="little")[:70].astype(bool)
    np.testing.assert_array_equal(unpacked, mask)


def test_acceleration_configuration_host_side():
    """HIPAccelerationConfiguration validates on the host; the backend
    choice takes the HIP device for .auto and keeps explicit choices."""
    from vectorstorekit_amd import DistanceComputeBackend, HIPAccelerationConfiguration

    HIPAccelerationConfiguration().validate()
    HIPAccelerationConfiguration.research().validate()
    with pytest.raises(vsk.VSKError):
        HIPAccelerationConfiguration(kernel="fast").validate()
    with pytest.raises(vsk.VSKError):
        HIPAccelerationConfiguration(maxTileBytes=-1).validate()
    B = DistanceComputeBackend
    assert B.auto.selectOptimal(128, 10) == B.hip
    assert B.auto.selectOptimal(512, 10, hipAvailable=False) == B.simd
    assert B.auto.selectOptimal(128, 5000, hipAvailable=False) == B.metal
    assert B.accelerate.selectOptimal(128, 5000) == B.accelerate
    lib = vsk.load_library()
    assert lib.vsk_configure(None, None) == -2

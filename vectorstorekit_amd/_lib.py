"""ctypes binding of libvsk_hip.so (the C ABI declared in include/vsk_hip.h).

The library is built in-tree (``vectorstorekit_amd/lib/libvsk_hip.so``) by
``__graft_entry__.build()`` / ``make -C vectorstorekit_amd/csrc``.  There is
no fallback: if the library is missing or cannot be loaded, every entry point
raises ``VSKError``.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char, c_char_p, c_double, c_float, c_int32, c_int64, c_void_p

import numpy as np

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libvsk_hip.so")

# status codes (vsk_hip.h)
VSK_OK = 0
STATUS_NAMES = {
    -1: "deviceNotAvailable",
    -2: "invalidArgument",
    -3: "emptyInput",
    -4: "dimensionMismatch",
    -5: "outOfMemory",
    -6: "executionFailed",
    -7: "notTrained",
    -8: "unsupportedOperation",
    -9: "invalidBufferSize",
    -10: "persistenceFailed",
}

# metric codes (vsk_hip.h)
METRIC_L2SQ = 0
METRIC_L2 = 1
METRIC_COSINE = 2
METRIC_COSINE_NORMALIZED = 3
METRIC_DOT = 4
METRIC_L1 = 5
METRIC_HAMMING = 6
METRIC_COSINE_NOEPS = 7
MAX_K = 1024
DB_NORMALIZE = 1


class VSKError(RuntimeError):
    """A failed C-ABI call: ``status`` is the vsk_status code, ``kind`` its
    name in the reference's error vocabulary."""

    def __init__(self, status: int, message: str):
        self.status = status
        self.kind = STATUS_NAMES.get(status, "unknown")
        super().__init__(f"{self.kind} ({status}): {message}")


class vsk_caps(ctypes.Structure):
    _fields_ = [
        ("name", c_char * 96),
        ("arch", c_char * 64),
        ("device", c_int32),
        ("compute_units", c_int32),
        ("wavefront_size", c_int32),
        ("lds_bytes_per_block", c_int32),
        ("global_mem_bytes", c_int64),
        ("clock_khz", c_int32),
        ("memory_clock_khz", c_int32),
        ("memory_bus_width_bits", c_int32),
    ]


class vsk_peaks(ctypes.Structure):
    _fields_ = [("bf16_tflops", c_double), ("int8_tops", c_double), ("hbm_gbs", c_double),
                ("hbm_read_gbs", c_double)]


class vsk_kernel_stat(ctypes.Structure):
    _fields_ = [("name", c_char * 64), ("launches", c_int64), ("total_ms", c_double),
                ("work", c_double)]


class vsk_config(ctypes.Structure):
    _fields_ = [("kernel", c_int32), ("enable_profiling", c_int32), ("max_tile_bytes", c_int64)]


KERNEL_AUTO, KERNEL_EXACT, KERNEL_SCREEN, KERNEL_BF16X3, KERNEL_FP32 = 0, 1, 2, 3, 4

P = c_void_p  # every buffer argument is passed as a raw address
PP = POINTER(c_void_p)

# name -> (restype, argtypes).  This table is the Python side of the ABI and
# must list every function of include/vsk_hip.h.
SIGNATURES = {
    "vsk_create": (c_int32, [c_int32, PP]),
    "vsk_destroy": (c_int32, [P]),
    "vsk_device_info": (c_int32, [P, POINTER(vsk_caps)]),
    "vsk_last_error": (c_char_p, [P]),
    "vsk_stream": (c_void_p, [P]),
    "vsk_last_kernel_ms": (c_float, [P]),
    "vsk_last_sync_count": (c_int32, [P]),
    "vsk_last_screen_redo": (c_int32, [P, c_int32, P, c_int64, P]),
    "vsk_measure_peaks": (c_int32, [P, POINTER(vsk_peaks)]),
    "vsk_configure": (c_int32, [P, POINTER(vsk_config)]),
    "vsk_get_config": (c_int32, [P, POINTER(vsk_config)]),
    "vsk_profile_enable": (c_int32, [P, c_int32]),
    "vsk_profile_only": (c_int32, [P, c_char_p]),
    "vsk_profile_reset": (c_int32, [P]),
    "vsk_profile_count": (c_int32, [P]),
    "vsk_profile_get": (c_int32, [P, c_int32, POINTER(vsk_kernel_stat)]),
    "vsk_db_upload_f32": (c_int32, [P, P, c_int64, c_int32, c_int32, PP]),
    "vsk_db_free": (c_int32, [P, P]),
    "vsk_db_info": (c_int32, [P, POINTER(c_int64), POINTER(c_int32)]),
    "vsk_db_read_f32": (c_int32, [P, P, c_int64, c_int64, P]),
    "vsk_search_flat": (c_int32, [P, P, P, c_int64, c_int32, c_int32, P, P]),
    "vsk_search_flat_filtered": (c_int32, [P, P, P, c_int64, c_int32, c_int32, P, c_int64, P,
                                           P]),
    "vsk_distances": (c_int32, [P, P, P, c_int64, c_int32, P]),
    "vsk_matrix_multiply": (c_int32, [P, P, c_int64, c_int32, P, c_int64, P]),
    "vsk_ivf_drop_rows": (c_int32, [P, P]),
    "vsk_ivf_storage": (c_int32, [P, P, P, P]),
    "vsk_ivf_create": (c_int32, [P, P, c_int32, c_int32, PP]),
    "vsk_ivf_free": (c_int32, [P, P]),
    "vsk_ivf_add": (c_int32, [P, P, P, P, c_int64]),
    "vsk_ivf_assign": (c_int32, [P, P, P, c_int64, P]),
    "vsk_ivf_probe": (c_int32, [P, P, P, c_int64, c_int32, P]),
    "vsk_ivf_search": (c_int32, [P, P, P, c_int64, c_int32, c_int32, c_int32, P, P]),
    "vsk_ivf_build": (c_int32, [P, P, c_int32, P, P, c_int64, c_int32, PP]),
    "vsk_ivf_list_sizes": (c_int32, [P, P, P]),
    "vsk_ivf_search_filtered": (c_int32, [P, P, P, c_int64, c_int32, c_int32, c_int32, P,
                                          c_int64, P, P]),
    "vsk_ivf_remove": (c_int32, [P, P, P, c_int64, P]),
    "vsk_ivf_list_ids": (c_int32, [P, P, P, P]),
    "vsk_ivf_encode_sq8": (c_int32, [P, P, c_int32, P, P]),
    "vsk_ivf_encode_pq": (c_int32, [P, P, P]),
    "vsk_ivf_save": (c_int32, [P, P, ctypes.c_char_p]),
    "vsk_ivf_load": (c_int32, [P, ctypes.c_char_p, PP]),
    "vsk_ivf_info": (c_int32, [P, P, P, P, P]),
    "vsk_ivf_set_meta": (c_int32, [P, P, P, c_int64]),
    "vsk_ivf_get_meta": (c_int32, [P, P, P, c_int64, P]),
    "vsk_ivf_centroids": (c_int32, [P, P, P]),
    "vsk_ivf_sq8_params": (c_int32, [P, P, P, P, P]),
    "vsk_ivf_search_sq8": (c_int32, [P, P, P, P, c_int64, c_int32, c_int32, P, P]),
    "vsk_ivf_search_pq": (c_int32, [P, P, P, P, c_int64, c_int32, c_int32, P, P]),
    "vsk_sq8_train": (c_int32, [P, P, c_int64, c_int32, c_int32, P, P]),
    "vsk_sq8_encode": (c_int32, [P, P, c_int64, c_int32, c_int32, P, P, P]),
    "vsk_scalar_quantize_u8": (c_int32, [P, P, c_int64, c_int32, c_int32, P, P, P]),
    "vsk_sq8_upload": (c_int32, [P, P, c_int64, c_int32, PP]),
    "vsk_sq8_free": (c_int32, [P, P]),
    "vsk_sq8_search": (c_int32, [P, P, P, c_int64, c_int32, P, P]),
    "vsk_sq8_search_noalloc": (c_int32, [P, P, P, c_int64, c_int32, P, P]),
    "vsk_pq_create": (c_int32, [P, P, c_int32, c_int32, c_int32, PP]),
    "vsk_pq_free": (c_int32, [P, P]),
    "vsk_pq_upload": (c_int32, [P, P, P, c_int64, c_int32, c_int32, PP]),
    "vsk_pq_encode": (c_int32, [P, P, P, c_int64, P]),
    "vsk_pq_add_codes": (c_int32, [P, P, P, c_int64]),
    "vsk_pq_lut": (c_int32, [P, P, P, c_int64, P]),
    "vsk_pq_search": (c_int32, [P, P, P, c_int64, c_int32, c_int32, c_int32, P, P, P]),
    "vsk_hnsw_distances": (c_int32, [P, P, P, c_int64, P, P, c_int32, P]),
    "vsk_kmeans": (c_int32, [P, P, c_int64, c_int32, c_int32, P, c_int32, P, ctypes.c_uint64,
                             c_int32, c_float, P, P, P]),
    "vsk_sq8_decode": (c_int32, [P, P, c_int64, c_int32, c_int32, P, P, P]),
    "vsk_pq_decode": (c_int32, [P, P, P, c_int64, P]),
    "vsk_binary_encode": (c_int32, [P, P, c_int64, c_int32, P]),
    "vsk_bin_upload": (c_int32, [P, P, c_int64, c_int32, PP]),
    "vsk_bin_free": (c_int32, [P, P]),
    "vsk_bin_search": (c_int32, [P, P, P, c_int64, c_int32, P, P]),
    "vsk_bin_distances": (c_int32, [P, P, P, c_int64, P]),
}

_lib = None


def library_path() -> str:
    return LIB_PATH


def load_library() -> ctypes.CDLL:
    """Load libvsk_hip.so once; raise VSKError when it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise VSKError(-1, f"native library not built: {LIB_PATH} is missing "
                       "(run __graft_entry__.build())")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        if not hasattr(lib, name):
            continue  # reported by exported_symbols() / the ABI test
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def exported_symbols() -> list[str]:
    """Names of SIGNATURES that the loaded library exports."""
    lib = load_library()
    return [n for n in SIGNATURES if hasattr(lib, n)]


# ---------------------------------------------------------------------------
# buffer marshalling: numpy arrays (host) or torch tensors (host or device)
# ---------------------------------------------------------------------------
def _is_torch(x) -> bool:
    return type(x).__module__.startswith("torch")


def as_buffer(x, dtype, shape=None):
    """Return (address, keepalive) for an input buffer of the given numpy
    dtype.  numpy inputs are converted/copied to C-contiguous as needed;
    torch tensors must already have the right dtype and be contiguous."""
    if _is_torch(x):
        import torch

        want = {np.float32: torch.float32, np.int64: torch.int64, np.int32: torch.int32,
                np.int8: torch.int8, np.uint8: torch.uint8}[np.dtype(dtype).type]
        if x.dtype != want:
            raise VSKError(-2, f"tensor dtype {x.dtype} != {want}")
        if not x.is_contiguous():
            x = x.contiguous()
        if shape is not None and tuple(x.shape) != tuple(shape):
            raise VSKError(-4, f"tensor shape {tuple(x.shape)} != {tuple(shape)}")
        return x.data_ptr(), x
    a = np.ascontiguousarray(x, dtype=dtype)
    if shape is not None and a.shape != tuple(shape):
        raise VSKError(-4, f"array shape {a.shape} != {tuple(shape)}")
    return a.ctypes.data, a


def out_buffer(shape, dtype, like=None):
    """Allocate an output buffer: a torch tensor on like's device when
    ``like`` is a CUDA tensor, else a numpy array."""
    if like is not None and _is_torch(like) and like.is_cuda:
        import torch

        tdt = {np.float32: torch.float32, np.int64: torch.int64, np.int32: torch.int32,
               np.int8: torch.int8, np.uint8: torch.uint8}[np.dtype(dtype).type]
        t = torch.empty(shape, dtype=tdt, device=like.device)
        return t.data_ptr(), t
    a = np.empty(shape, dtype=dtype)
    return a.ctypes.data, a


def row_bitmap(allowed, nbits: int | None = None) -> np.ndarray:
    """A row filter as the C ABI takes it: bit i (bit i % 32 of word i // 32)
    is set when row (or id) i may be a candidate.  ``allowed`` is a boolean
    array over the rows or an iterable of the allowed indices (then nbits
    gives the bitmap's length)."""
    a = np.asarray(allowed)
    if a.dtype == np.bool_:
        bits = a.reshape(-1)
    else:
        n = int(nbits if nbits is not None else (a.max() + 1 if a.size else 0))
        bits = np.zeros(n, np.bool_)
        if a.size:
            bits[a.astype(np.int64)] = True
    words = np.packbits(bits, bitorder="little")
    pad = (-words.size) % 4
    if pad:
        words = np.concatenate([words, np.zeros(pad, np.uint8)])
    return words.view(np.uint32)


def check(ctx_handle, status: int):
    if status != VSK_OK:
        lib = load_library()
        msg = lib.vsk_last_error(ctx_handle)
        raise VSKError(status, msg.decode() if msg else "")

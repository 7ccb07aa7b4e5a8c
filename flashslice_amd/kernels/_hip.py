"""ctypes binding of the HIP library's C ABI (``include/flashslice_hip.h``).

The library is ``flashslice_amd/_lib/libflashslice_hip.so``, built in-tree by
``python -m flashslice_amd.build``. It is loaded lazily, once, under a lock,
after ``torch`` (so it binds to the HIP runtime torch already loaded). There
is no CPU fallback: if the library is missing, every op raises.
"""

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                        "_lib", "libflashslice_hip.so")

FS_OK, FS_ERR_INVALID, FS_ERR_UNSUPPORTED, FS_ERR_WORKSPACE, FS_ERR_HIP = range(5)
OP_SLICE_FWD, OP_DESLICE_FWD, OP_SLICE_BWD, OP_DESLICE_BWD, OP_STATS, OP_TIED_BWD = range(6)

_DTYPES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}

#: every entry point the header declares
EXPORTS = ("fs_workspace_bytes", "fs_compute_stats", "fs_slice_fwd", "fs_deslice_fwd",
           "fs_slice_bwd", "fs_deslice_bwd", "fs_tied_bwd", "fs_family", "fs_last_error",
           "fs_version", "fs_slice_fwd_static",
           # the layer around the path (include/flashslice_layer.h)
           "fs_layernorm_fwd", "fs_layernorm_bwd", "fs_layernorm_workspace_bytes")


class FsPoints(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p),
                ("stride_b", ctypes.c_int64), ("stride_n", ctypes.c_int64),
                ("stride_h", ctypes.c_int64),
                ("dtype", ctypes.c_int32), ("width", ctypes.c_int32)]


class FsSliceParams(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int64), ("N", ctypes.c_int64), ("H", ctypes.c_int64),
                ("D", ctypes.c_int64), ("DV", ctypes.c_int64), ("G", ctypes.c_int64),
                ("weight", ctypes.c_void_p),
                ("w_stride_b", ctypes.c_int64), ("w_stride_h", ctypes.c_int64),
                ("bias", ctypes.c_void_p),
                ("b_stride_b", ctypes.c_int64), ("b_stride_h", ctypes.c_int64),
                ("tau", ctypes.c_void_p),
                ("dot", ctypes.c_int32), ("family", ctypes.c_int32),
                ("row_splits", ctypes.c_void_p), ("total_rows", ctypes.c_int64)]


class FlashSliceLibError(RuntimeError):
    """A failure reported by the HIP library (its fs_last_error text)."""


_LIB = None
_LOCK = threading.Lock()


def _declare(lib):
    P, V, S, I32 = ctypes.POINTER, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int32
    pts, prm = P(FsPoints), P(FsSliceParams)
    lib.fs_workspace_bytes.argtypes = [I32, prm]
    lib.fs_workspace_bytes.restype = S
    lib.fs_compute_stats.argtypes = [pts, prm, V, I32, V, S, V]
    lib.fs_slice_fwd.argtypes = [pts, pts, prm, V, V, V, V, V, S, V]
    lib.fs_slice_fwd_static.argtypes = [pts, pts, prm, V, V, V, V, V]
    lib.fs_deslice_fwd.argtypes = [pts, prm, V, V, V, pts, V, S, V]
    lib.fs_slice_bwd.argtypes = [pts, pts, prm, V, V, V, pts, pts, V, V, V, V, S, V]
    lib.fs_deslice_bwd.argtypes = [pts, prm, V, V, pts, pts, V, V, V, V, V, S, V]
    lib.fs_tied_bwd.argtypes = [pts, pts, pts, prm, V, V, V, pts, pts, V, V, V, V, V, S, V]
    for name in ("fs_compute_stats", "fs_slice_fwd", "fs_deslice_fwd", "fs_slice_bwd",
                 "fs_deslice_bwd", "fs_tied_bwd", "fs_slice_fwd_static"):
        getattr(lib, name).restype = I32
    lib.fs_family.argtypes = [prm]
    lib.fs_family.restype = I32
    lib.fs_last_error.argtypes = []
    lib.fs_last_error.restype = ctypes.c_char_p
    lib.fs_version.argtypes = []
    lib.fs_version.restype = ctypes.c_char_p
    I64, F32 = ctypes.c_int64, ctypes.c_float
    lib.fs_layernorm_fwd.argtypes = [V, V, V, V, V, V, I64, I32, F32, V]
    lib.fs_layernorm_fwd.restype = I32
    lib.fs_layernorm_workspace_bytes.argtypes = [I64, I32]
    lib.fs_layernorm_workspace_bytes.restype = S
    lib.fs_layernorm_bwd.argtypes = [V, V, V, V, V, V, V, V, V, S, I64, I32, V]
    lib.fs_layernorm_bwd.restype = I32


def lib():
    """The loaded library (loads it on first use). Raises if it is missing."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is None:
            if not os.path.exists(LIB_PATH):
                raise FlashSliceLibError(
                    "flashslice_amd: the HIP library %s is not built; run "
                    "`python -m flashslice_amd.build` (there is no CPU fallback)" % LIB_PATH)
            handle = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_LOCAL)
            _declare(handle)
            _LIB = handle
    return _LIB


def check(rc):
    if rc != FS_OK:
        msg = lib().fs_last_error().decode()
        if rc == FS_ERR_INVALID:
            raise ValueError(msg)
        raise FlashSliceLibError(msg)


def dtype_code(t):
    return _DTYPES.get(t.dtype)


def points(t, width):
    """FsPoints of a (B, N, H, width) tensor with unit stride on the last dim
    (a (1, rows, H, width) view of a ragged batch's points: its stride along
    b is not used)."""
    assert t.dim() == 4 and t.stride(3) == 1 and t.dtype in _DTYPES
    return FsPoints(t.data_ptr(), t.stride(0), t.stride(1), t.stride(2), _DTYPES[t.dtype], width)


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)

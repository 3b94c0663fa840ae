"""ctypes binding of ``order.c`` (test infrastructure only)."""

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "liborder.so")
_lib = None


def build():
    subprocess.run(["make", "-s", "-B", "-C", _HERE, "liborder.so"], check=True)


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            build()
        lib = ctypes.CDLL(_LIB)
        lib.oracle_row_sums_f32.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
        lib.oracle_sum_1d_f32.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int]
        lib.oracle_sum_1d_f32.restype = ctypes.c_float
        lib.oracle_categorical_rows.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                                ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        _lib = lib
    return _lib


def row_sums(x):
    """fp32 row sums of a 2-D array in torch-CPU cascade order."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape[0], dtype=np.float32)
    _load().oracle_row_sums_f32(x.ctypes.data, x.shape[0], x.shape[1], out.ctypes.data)
    return out


def sum_1d(x, threads):
    """fp32 ``x.sum()`` of a 1-D array as torch-CPU computes it with ``threads`` threads."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    return np.float32(_load().oracle_sum_1d_f32(x.ctypes.data, x.shape[0], int(threads)))


def categorical(w, u):
    """Sequential-fp64 inverse-CDF draw per row (slow: O(V log V))."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    idx = np.empty(w.shape[0], dtype=np.int64)
    valid = np.empty(w.shape[0], dtype=np.uint8)
    _load().oracle_categorical_rows(w.ctypes.data, w.shape[0], w.shape[1], u.ctypes.data,
                                    idx.ctypes.data, valid.ctypes.data)
    return idx, valid.astype(bool)

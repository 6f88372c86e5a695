"""ctypes loader for the C restatement ``lowbit_ref.c`` (test infrastructure only)."""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB = _HERE / "liblowbit_ref.so"
_lib = None


def build() -> Path:
    """Compile ``lowbit_ref.c`` with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB


def lib():
    global _lib
    if _lib is None:
        if not _LIB.exists():
            build()
        _lib = ctypes.CDLL(str(_LIB))
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        _lib.orc_rowwise_value.argtypes = [P, I64, ctypes.c_int, ctypes.c_int]
        _lib.orc_rowwise_value.restype = ctypes.c_int
        _lib.orc_rowwise_gemm.argtypes = [P, I64, I64, P, I64, P, I64, I64, I64, I64, ctypes.c_int, P]
        _lib.orc_rowwise_gemm.restype = None
        _lib.orc_marlin_code.argtypes = [P, I64, I64, I64]
        _lib.orc_marlin_code.restype = ctypes.c_int
        _lib.orc_marlin_scale.argtypes = [P, I64, I64, I64, ctypes.c_int]
        _lib.orc_marlin_scale.restype = ctypes.c_uint16
        _lib.orc_marlin_gemm.argtypes = [P, I64, P, P, I64, I64, I64, P, I64, P]
        _lib.orc_marlin_gemm.restype = None
        _lib.orc_marlin_inverse_tables.argtypes = [P, P, P]
        _lib.orc_marlin_inverse_tables.restype = None
        _lib.orc_float_to_half.argtypes = [ctypes.c_float]
        _lib.orc_float_to_half.restype = ctypes.c_uint16
        _lib.orc_half_to_float.argtypes = [ctypes.c_uint16]
        _lib.orc_half_to_float.restype = ctypes.c_float
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def rowwise_gemm(packed, scales, x, cols, group_size, bits) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float16)
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float16)
    rows = packed.shape[0]
    y = np.empty((x.shape[0], rows), dtype=np.float16)
    lib().orc_rowwise_gemm(_p(packed), rows, packed.shape[1], _p(scales), scales.shape[1],
                           _p(x), x.shape[0], x.shape[1], cols, group_size, bits, _p(y))
    return y


def marlin_gemm(x, qweight, scales, group_size, rows=None) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float16)
    qweight = np.ascontiguousarray(qweight, dtype=np.int32)
    scales = np.ascontiguousarray(scales, dtype=np.float16)
    m, k = x.shape
    n = qweight.shape[1] // 2
    if rows is None:
        ridx, nrows = None, m
    else:
        ridx = np.ascontiguousarray(rows, dtype=np.int64)
        nrows = ridx.size
    out = np.empty((nrows, n), dtype=np.float16)
    lib().orc_marlin_gemm(_p(x), m, _p(qweight), _p(scales), n, k, group_size,
                          None if ridx is None else _p(ridx), nrows, _p(out))
    return out


def marlin_inverse_tables():
    a = np.empty(1024, dtype=np.int32)
    b = np.empty(64, dtype=np.int32)
    c = np.empty(32, dtype=np.int32)
    lib().orc_marlin_inverse_tables(_p(a), _p(b), _p(c))
    return a, b, c

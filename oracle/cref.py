"""ctypes loader for oracle/_build/libvt_oracle.so (test infrastructure only).

Wraps the C restatement in ref_gemm.c: vt_ref_gemm_i8 (the emitted
`veritac_scalar_ref` loop order, backend.py:712-720) and vt_ref_gemm_i8_ikj
(same function, i-t-j order), plus the C lcg filler (backend.py:738-746).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libvt_oracle.so")
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def load(build_if_missing=True):
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        if not build_if_missing:
            raise FileNotFoundError(LIB_PATH)
        build()
    lib = ctypes.CDLL(LIB_PATH)
    p = ctypes.c_void_p
    i64 = ctypes.c_int64
    for name in ("vt_ref_gemm_i8", "vt_ref_gemm_i8_ikj"):
        fn = getattr(lib, name)
        fn.argtypes = [p, p, p, p, i64, i64, i64, i64, i64, i64, i64, ctypes.c_int]
        fn.restype = None
    lib.vt_ref_lcg_fill.argtypes = [ctypes.c_uint32, p, i64, p, i64]
    lib.vt_ref_lcg_fill.restype = None
    lib.vt_ref_threads.argtypes = []
    lib.vt_ref_threads.restype = ctypes.c_int
    _lib = lib
    return lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def gemm_i8(A, B, D=None, threads=0, order="ijk", out=None):
    """C = D + A.B (int32, wrapping) for 2-D row-major contiguous operands."""
    lib = load()
    A = np.ascontiguousarray(A, dtype=np.int8)
    B = np.ascontiguousarray(B, dtype=np.int8)
    M, K = A.shape
    K2, N = B.shape
    if K != K2:
        raise ValueError("inner dimensions differ")
    if D is not None:
        D = np.ascontiguousarray(D, dtype=np.int32)
        if D.shape != (M, N):
            raise ValueError("D must be M x N")
    C = out if out is not None else np.empty((M, N), dtype=np.int32)
    fn = lib.vt_ref_gemm_i8 if order == "ijk" else lib.vt_ref_gemm_i8_ikj
    fn(_ptr(A), _ptr(B), _ptr(D), _ptr(C), M, N, K, K, N, N, N, int(threads))
    return C


def lcg_fill(seed, size_a, size_b):
    lib = load()
    A = np.empty(size_a, dtype=np.int8)
    B = np.empty(size_b, dtype=np.int8)
    lib.vt_ref_lcg_fill(seed & 0xFFFFFFFF, _ptr(A), size_a, _ptr(B), size_b)
    return A, B


def threads():
    return load().vt_ref_threads()

"""ctypes loader for the oracle's C libraries (test infrastructure only).

Wraps the C restatement in ref_gemm.c: vt_ref_gemm_i8 (the emitted
`veritac_scalar_ref` loop order, backend.py:712-720) and vt_ref_gemm_i8_ikj
(same function, i-t-j order), the C lcg filler (backend.py:738-746), and the
reference's own CPU GEMM, the stride-1000 double loop nest
(vt_ref_matmul_f64_stride1000, emit_c.py:29-155).

The same source is built three ways (oracle/Makefile): "default"
(-O3 x86-64-v3), "O2" (the reference runner's -O2 -fopenmp, runner.py:48)
and "v4" (-O3 x86-64-v4, AVX-512; loaded only where host_has_avx512()).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libvt_oracle.so")
BUILDS = {"default": LIB_PATH,
          "O2": os.path.join(_HERE, "_build", "libvt_oracle_O2.so"),
          "v4": os.path.join(_HERE, "_build", "libvt_oracle_v4.so")}
_libs = {}


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def host_has_avx512():
    """True when this host's CPU reports the AVX-512 subsets x86-64-v4 needs."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    flags = set(line.split(":", 1)[1].split())
                    return {"avx512f", "avx512bw", "avx512dq", "avx512vl"} <= flags
    except OSError:
        pass
    return False


def load(build_if_missing=True, variant="default"):
    if variant in _libs:
        return _libs[variant]
    if variant not in BUILDS:
        raise ValueError("unknown oracle build %r" % (variant,))
    if variant == "v4" and not host_has_avx512():
        raise RuntimeError("the x86-64-v4 oracle build needs AVX-512, which this host lacks")
    path = BUILDS[variant]
    if not os.path.exists(path):
        if not build_if_missing:
            raise FileNotFoundError(path)
        build()
    lib = ctypes.CDLL(path)
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
    lib.vt_ref_matmul_f64_stride1000.argtypes = [p, p, p, i64, i64, i64]
    lib.vt_ref_matmul_f64_stride1000.restype = None
    _libs[variant] = lib
    return lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def gemm_i8(A, B, D=None, threads=0, order="ijk", out=None, variant="default"):
    """C = D + A.B (int32, wrapping) for 2-D row-major contiguous operands."""
    lib = load(variant=variant)
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


def matmul_f64_stride1000(A_flat, B_flat, C_flat, M, K, N, variant="default"):
    """C += A.B over flat float64 buffers in the stride-1000 layout (in place)."""
    if max(M, K, N) > 1000:
        raise ValueError("the stride-1000 layout needs M, K, N <= 1000")
    need = {"A": (M - 1) * 1000 + K, "B": (K - 1) * 1000 + N, "C": (M - 1) * 1000 + N}
    for name, buf in (("A", A_flat), ("B", B_flat), ("C", C_flat)):
        if buf.dtype != np.float64 or not buf.flags.c_contiguous or buf.size < need[name]:
            raise ValueError("%s must be a contiguous float64 buffer of >= %d cells"
                             % (name, need[name]))
    load(variant=variant).vt_ref_matmul_f64_stride1000(_ptr(A_flat), _ptr(B_flat), _ptr(C_flat),
                                                       M, K, N)
    return C_flat


def lcg_fill(seed, size_a, size_b):
    lib = load()
    A = np.empty(size_a, dtype=np.int8)
    B = np.empty(size_b, dtype=np.int8)
    lib.vt_ref_lcg_fill(seed & 0xFFFFFFFF, _ptr(A), size_a, _ptr(B), size_b)
    return A, B


def threads():
    return load().vt_ref_threads()

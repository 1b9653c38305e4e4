"""ctypes binding of libvt_hip_gemm.so (declarations in include/vt_hip_gemm.h).

The library path is veritac_amd/libvt_hip_gemm.so unless the VT_HIP_GEMM_LIB
environment variable names another file (the analogue of the reference's
VERITAC_GEMMINI_CHECK_BIN override, specializations/gemmini_gemm/
backend.py:156-161). A missing or unloadable library raises HipGemmError:
there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os
import threading

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
DEFAULT_LIB = os.path.join(PKG_DIR, "libvt_hip_gemm.so")
ABI_VERSION = 7

VT_OK = 0
VT_EINVAL = -1
VT_EUNSUPPORTED = -2
VT_EHIP = -3
VT_ENODEV = -4
STATUS_NAMES = {VT_OK: "ok", VT_EINVAL: "invalid argument", VT_EUNSUPPORTED: "unsupported",
                VT_EHIP: "HIP error", VT_ENODEV: "no gfx950 device"}

# variant name -> id (include/vt_hip_gemm.h VT_VARIANT_*)
VARIANT_IDS = {
    "auto": 0,
    "mfma_256x256": 1,
    "mfma_128x128": 2,
    "skinny": 3,
    "generic": 4,
    "mfma_256x128": 5,
    "padded": 6,
}
VARIANTS = tuple(VARIANT_IDS)

# Every function include/vt_hip_gemm.h declares.
EXPORTS = ("vt_gemm_i8", "vt_gemm_i8_noalloc", "vt_gemm_check", "vt_gemm_select", "vt_variant_info", "vt_variant_name",
           "vt_last_error", "vt_sync", "vt_device_count", "vt_abi_version", "vt_replay_i8",
           "vt_device_query", "vt_packed_b_size", "vt_pack_b_i8", "vt_gemm_i8_packed",
           "vt_rtc_compile", "vt_rtc_code_size", "vt_rtc_launch", "vt_rtc_release")

# Replay operation codes and status codes (VT_REPLAY_* in include/vt_hip_gemm.h).
REPLAY_MVIN, REPLAY_LATCH_B, REPLAY_COMPUTE, REPLAY_MVOUT = 1, 2, 3, 4
REPLAY_STATUS = {0: "ok", 1: "int32 accumulator overflow", 2: "operand out of range",
                 3: "unknown operation"}


class DeviceInfo(ctypes.Structure):
    """vt_device_info of include/vt_hip_gemm.h (field for field)."""
    _fields_ = [
        ("name", ctypes.c_char * 256),
        ("arch", ctypes.c_char * 256),
        ("code_object_arch", ctypes.c_char * 32),
        ("total_memory_bytes", ctypes.c_int64),
        ("l2_cache_bytes", ctypes.c_int64),
        ("lds_per_workgroup_bytes", ctypes.c_int64),
        ("lds_per_cu_bytes", ctypes.c_int64),
        ("compute_units", ctypes.c_int32),
        ("wavefront_size", ctypes.c_int32),
        ("max_threads_per_workgroup", ctypes.c_int32),
        ("max_clock_khz", ctypes.c_int32),
        ("memory_clock_khz", ctypes.c_int32),
        ("memory_bus_width_bits", ctypes.c_int32),
        ("pci_domain", ctypes.c_int32),
        ("pci_bus", ctypes.c_int32),
        ("pci_device", ctypes.c_int32),
        ("hip_runtime_version", ctypes.c_int32),
        ("hip_driver_version", ctypes.c_int32),
        ("supported", ctypes.c_int32),
    ]


class HipGemmError(RuntimeError):
    """Raised by the hip_gemm boundary on any refusal or device failure."""

    def __init__(self, message, code=None):
        super().__init__(message)
        self.code = code


_lock = threading.Lock()
_lib = None


def library_path():
    return os.environ.get("VT_HIP_GEMM_LIB") or DEFAULT_LIB


def _declare(lib):
    i64, i32, p = ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p
    pi32 = ctypes.POINTER(ctypes.c_int32)
    lib.vt_gemm_i8.argtypes = [p, p, p, p, i64, i64, i64, i64, i64, i64, i64,
                               i64, i64, i64, i64, i64, i32, i32, p]
    lib.vt_gemm_i8.restype = ctypes.c_int
    lib.vt_gemm_i8_noalloc.argtypes = lib.vt_gemm_i8.argtypes
    lib.vt_gemm_i8_noalloc.restype = ctypes.c_int
    lib.vt_gemm_check.argtypes = [i64] * 12 + [i32, i32, i32, pi32, pi32,
                                                ctypes.POINTER(ctypes.c_int64)]
    lib.vt_gemm_check.restype = ctypes.c_int
    lib.vt_gemm_select.argtypes = [i64, i64, i64, i64, i64, i64, i32, pi32, pi32]
    lib.vt_gemm_select.restype = ctypes.c_int
    lib.vt_variant_info.argtypes = [i32, pi32, pi32, pi32, pi32, pi32]
    lib.vt_variant_info.restype = ctypes.c_int
    lib.vt_variant_name.argtypes = [i32]
    lib.vt_variant_name.restype = ctypes.c_char_p
    lib.vt_last_error.argtypes = []
    lib.vt_last_error.restype = ctypes.c_char_p
    lib.vt_sync.argtypes = [p]
    lib.vt_sync.restype = ctypes.c_int
    lib.vt_device_count.argtypes = []
    lib.vt_device_count.restype = ctypes.c_int
    lib.vt_replay_i8.argtypes = [p, i64, p, p, p, i64, i64, i64, i64, i64, p, p]
    lib.vt_replay_i8.restype = ctypes.c_int
    lib.vt_device_query.argtypes = [i32, ctypes.POINTER(DeviceInfo), i64]
    lib.vt_device_query.restype = ctypes.c_int
    lib.vt_abi_version.argtypes = []
    lib.vt_abi_version.restype = ctypes.c_int
    lib.vt_packed_b_size.argtypes = [i64, i64]
    lib.vt_packed_b_size.restype = ctypes.c_int64
    lib.vt_pack_b_i8.argtypes = [p, p, i64, i64, i64, i64, i64, i64, p]
    lib.vt_pack_b_i8.restype = ctypes.c_int
    lib.vt_gemm_i8_packed.argtypes = [p, p, p, p, i64, i64, i64, i64, i64, i64, i64,
                                      i64, i64, i64, i64, i32, p]
    lib.vt_gemm_i8_packed.restype = ctypes.c_int
    lib.vt_rtc_compile.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(p)]
    lib.vt_rtc_compile.restype = ctypes.c_int
    lib.vt_rtc_code_size.argtypes = [p]
    lib.vt_rtc_code_size.restype = ctypes.c_int64
    u32 = ctypes.c_uint32
    lib.vt_rtc_launch.argtypes = [p, u32, u32, u32, u32, u32, u32, ctypes.POINTER(p), p]
    lib.vt_rtc_launch.restype = ctypes.c_int
    lib.vt_rtc_release.argtypes = [p]
    lib.vt_rtc_release.restype = None


def load_library():
    """Load (once) and return the native library; raise HipGemmError if absent."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not os.path.isfile(path):
            raise HipGemmError("libvt_hip_gemm.so not found at %r (build it with "
                               "`python -m veritac_amd.build`)" % path, VT_ENODEV)
        try:
            lib = ctypes.CDLL(path)
        except OSError as exc:
            raise HipGemmError("cannot load %r: %s" % (path, exc), VT_ENODEV) from exc
        missing = [n for n in EXPORTS if not hasattr(lib, n)]
        if missing:
            raise HipGemmError("%r lacks symbols %s" % (path, missing), VT_ENODEV)
        _declare(lib)
        if lib.vt_abi_version() != ABI_VERSION:
            raise HipGemmError("ABI version %d != %d" % (lib.vt_abi_version(), ABI_VERSION))
        _lib = lib
        return lib


def last_error():
    msg = load_library().vt_last_error()
    return msg.decode() if msg else ""


def check(status, what="vt_gemm_i8"):
    if status != VT_OK:
        raise HipGemmError("%s: %s (%s)" % (what, last_error(), STATUS_NAMES.get(status, status)),
                           status)
    return status


SELECT_ALIGNED, SELECT_B_SHARED = 1, 2   # vt_gemm_select flags


def select_variant(m, n, k, batch=1, lda=None, ldb=None, aligned=True, b_shared=False):
    """(variant name, k_split) that VT_VARIANT_AUTO launches for this shape
    (contiguous operands; b_shared: one B for every batch)."""
    lib = load_library()
    v, ks = ctypes.c_int32(), ctypes.c_int32()
    flags = (SELECT_ALIGNED if aligned else 0) | (SELECT_B_SHARED if b_shared else 0)
    check(lib.vt_gemm_select(m, n, k, batch, k if lda is None else lda,
                             n if ldb is None else ldb, flags,
                             ctypes.byref(v), ctypes.byref(ks)), "vt_gemm_select")
    names = {i: nm for nm, i in VARIANT_IDS.items()}
    return names[v.value], ks.value


def gemm_check(M, N, K, lda, ldb, ldd, ldc, batch=1, stride_a=0, stride_b=0, stride_d=0,
               stride_c=0, has_d=False, variant="auto", k_split=0):
    """vt_gemm_check: (status, reason, variant name, k_split, workspace bytes).

    Never raises for a refusal: status is VT_OK or the VT_E* code vt_gemm_i8
    would return, reason the native message. Loading the library can raise
    HipGemmError (the caller decides how to fail closed).
    """
    lib = load_library()
    vid = VARIANT_IDS[variant] if isinstance(variant, str) else int(variant)
    v, ks, ws = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64()
    st = lib.vt_gemm_check(M, N, K, lda, ldb, ldd, ldc, batch, stride_a, stride_b, stride_d,
                           stride_c, int(bool(has_d)), vid, k_split, ctypes.byref(v),
                           ctypes.byref(ks), ctypes.byref(ws))
    if st != VT_OK:
        return st, last_error(), None, None, None
    names = {i: nm for nm, i in VARIANT_IDS.items()}
    return st, "ok", names[v.value], ks.value, ws.value


def variant_info(name):
    """Static resources of a variant: tile_m, tile_n, tile_k, threads, lds_bytes."""
    lib = load_library()
    vals = [ctypes.c_int32() for _ in range(5)]
    check(lib.vt_variant_info(VARIANT_IDS[name], *[ctypes.byref(v) for v in vals]),
          "vt_variant_info")
    return dict(zip(("tile_m", "tile_n", "tile_k", "threads", "lds_bytes"),
                    (v.value for v in vals)))


def device_count():
    return load_library().vt_device_count()


def gemm_raw(A_ptr, B_ptr, D_ptr, C_ptr, M, N, K, lda, ldb, ldd, ldc, batch=1,
             stride_a=0, stride_b=0, stride_d=0, stride_c=0, variant="auto",
             k_split=0, stream=None):
    """One vt_gemm_i8 call on raw device pointers (integers); raises on failure."""
    lib = load_library()
    vid = VARIANT_IDS[variant] if isinstance(variant, str) else int(variant)
    st = lib.vt_gemm_i8(A_ptr, B_ptr, D_ptr, C_ptr, M, N, K, lda, ldb, ldd, ldc, batch,
                        stride_a, stride_b, stride_d, stride_c, vid, k_split, stream)
    return check(st)


NOALLOC_SCRATCH_BYTES = 32 << 20   # VT_NOALLOC_SCRATCH_BYTES


def gemm_noalloc_raw(A_ptr, B_ptr, D_ptr, C_ptr, M, N, K, lda, ldb, ldd, ldc, batch=1,
                     stride_a=0, stride_b=0, stride_d=0, stride_c=0, variant="auto",
                     k_split=0, stream=None):
    """One vt_gemm_i8_noalloc call (scratch from the static array, no
    allocation) on raw device pointers; raises on failure."""
    lib = load_library()
    vid = VARIANT_IDS[variant] if isinstance(variant, str) else int(variant)
    st = lib.vt_gemm_i8_noalloc(A_ptr, B_ptr, D_ptr, C_ptr, M, N, K, lda, ldb, ldd, ldc, batch,
                                stride_a, stride_b, stride_d, stride_c, vid, k_split, stream)
    return check(st, "vt_gemm_i8_noalloc")


def sync(stream=None):
    return check(load_library().vt_sync(stream), "vt_sync")


def replay_raw(prog_ptr, n_ops, A_ptr, B_ptr, C_ptr, m, n, k, scratchpad_rows,
               accumulator_rows, status_ptr, stream=None):
    """One vt_replay_i8 call on raw device pointers (integers); raises on failure.

    The device-side outcome is written to the 4-word status buffer; read it
    after synchronizing the stream.
    """
    lib = load_library()
    check(lib.vt_replay_i8(prog_ptr, n_ops, A_ptr, B_ptr, C_ptr, m, n, k, scratchpad_rows,
                           accumulator_rows, status_ptr, stream), "vt_replay_i8")


def device_query(device=-1):
    """vt_device_query as a dict of plain values; raises HipGemmError on refusal
    (VT_ENODEV on a host without HIP devices)."""
    lib = load_library()
    info = DeviceInfo()
    check(lib.vt_device_query(device, ctypes.byref(info), ctypes.sizeof(info)),
          "vt_device_query")
    out = {}
    for name, _ in DeviceInfo._fields_:
        v = getattr(info, name)
        out[name] = v.decode("utf-8", "replace") if isinstance(v, bytes) else int(v)
    return out


def packed_b_size(k, n):
    """Bytes of one packed B (vt_packed_b_size); raises for shapes the format refuses."""
    size = load_library().vt_packed_b_size(k, n)
    if size < 0:
        check(int(size), "vt_packed_b_size")
    return size


def pack_b_raw(B_ptr, Bp_ptr, K, N, ldb, batch=1, stride_b=0, stride_bp=0, stream=None):
    """One vt_pack_b_i8 call on raw device pointers (integers); raises on failure."""
    lib = load_library()
    return check(lib.vt_pack_b_i8(B_ptr, Bp_ptr, K, N, ldb, batch, stride_b, stride_bp, stream),
                 "vt_pack_b_i8")


def gemm_packed_raw(A_ptr, Bp_ptr, D_ptr, C_ptr, M, N, K, lda, ldd, ldc, batch=1,
                    stride_a=0, stride_bp=0, stride_d=0, stride_c=0, k_split=0, stream=None):
    """One vt_gemm_i8_packed call on raw device pointers (integers); raises on failure."""
    lib = load_library()
    st = lib.vt_gemm_i8_packed(A_ptr, Bp_ptr, D_ptr, C_ptr, M, N, K, lda, ldd, ldc, batch,
                               stride_a, stride_bp, stride_d, stride_c, k_split, stream)
    return check(st, "vt_gemm_i8_packed")


class RtcProgram:
    """A kernel compiled at run time by vt_rtc_compile (freed with the object)."""

    def __init__(self, source, kernel_name):
        lib = load_library()
        handle = ctypes.c_void_p()
        check(lib.vt_rtc_compile(source.encode(), kernel_name.encode(), ctypes.byref(handle)),
              "vt_rtc_compile")
        self._lib, self._handle, self.kernel_name = lib, handle, kernel_name

    @property
    def code_size(self):
        return self._lib.vt_rtc_code_size(self._handle)

    def launch(self, grid, block, arg_values, stream=None):
        """Launch with `arg_values`: ctypes scalars or pointers, one per kernel
        parameter in order (kept alive for the call)."""
        ptrs = (ctypes.c_void_p * max(1, len(arg_values)))(
            *[ctypes.cast(ctypes.byref(v), ctypes.c_void_p) for v in arg_values])
        g = tuple(grid) + (1,) * (3 - len(grid))
        b = tuple(block) + (1,) * (3 - len(block))
        check(self._lib.vt_rtc_launch(self._handle, *g, *b, ptrs, stream), "vt_rtc_launch")

    def close(self):
        if self._handle:
            self._lib.vt_rtc_release(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

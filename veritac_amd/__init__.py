"""veritac_amd -- MI355X (gfx950) exact int8 x int8 -> int32 GEMM.

The hot path of VeriTac's Gemmini GEMM contract, rebuilt as hand-written HIP
kernels behind a C ABI (include/vt_hip_gemm.h, libvt_hip_gemm.so), bound with
ctypes, and exposed as the `hip_gemm` specialization
(veritac_amd.specializations.hip_gemm) with the reference's
candidate / validate / run / benchmark interface.

Importing the package loads nothing native: the names below resolve lazily so
that listing the specialization catalog stays standard-library only.
"""

__all__ = ["HipGemmError", "load_library", "library_path", "VARIANTS", "VARIANT_IDS"]


def __getattr__(name):
    if name in __all__:
        from . import _lib
        return getattr(_lib, name)
    raise AttributeError(name)

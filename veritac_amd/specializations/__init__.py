"""Specialization catalog of this package (cf. the reference's specializations/).

Importing this package or listing the catalog imports only the standard
library; the hip_gemm backend (numpy, torch, the native library) is imported
only when used.
"""

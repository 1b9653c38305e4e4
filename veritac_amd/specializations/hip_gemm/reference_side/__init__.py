"""hip_gemm: exact int8 x int8 -> int32 GEMM on AMD MI355X (gfx950).

This directory is copied into a reference checkout as
specializations/hip_gemm/. Its modules re-export the hip_gemm backend of the
veritac_amd package, a separate checkout named by the VT_HIP_GEMM_REPO
environment variable (see _locate.py).
"""

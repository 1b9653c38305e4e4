"""hip_gemm: exact int8 x int8 -> int32 GEMM on MI355X (gfx950).

Import the submodules explicitly: backend (plans, validation, optimize, run),
runner (benchmark_gemm), inputs (deterministic generators).
"""

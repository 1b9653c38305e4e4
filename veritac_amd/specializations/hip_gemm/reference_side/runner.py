"""hip_gemm benchmark verb, reference side: the analogue of
specializations/cpu_gemm/runner.py:benchmark_matmul (same keys, with
gpu_time_ms in place of c_time_ms and cpu_time_ms in place of
numpy_time_ms)."""
from ._locate import add_repo_to_path

add_repo_to_path()

from veritac_amd.specializations.hip_gemm.runner import benchmark_gemm  # noqa: E402,F401

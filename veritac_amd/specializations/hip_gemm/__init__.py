"""hip_gemm: exact int8 x int8 -> int32 GEMM on MI355X (gfx950).

Import the submodules explicitly (none loads the native library at import):
  backend     plans, validation, optimize, run, packed-B weights (pack_b)
  runner      benchmark_gemm (the reference runner's benchmark dict)
  inputs      deterministic generators and the benchmark configurations
  replay      Gemmini command streams executed on the GPU
  loopnest    loop-nest JSON emitted as HIP kernels, compiled at run time
  provenance  hardware profile and hash-bound run reports
  verify      exact GPU-side check C == D + A.B (mod 2^32)
"""

"""hip_gemm backend, reference side: the verbs of
specializations/gemmini_gemm/backend.py for the MI355X GEMM.

make_plan, required_resources, validate_plan, gen_candidates, modeled_counts,
modeled_objective, optimize (candidates carry check{accepted, reason}, as in
backend.py:1083-1091), run / run_flat, which raise HipGemmError where
run_commands raises GemminiError, and emit_c / sha256_file (a standalone
self-checking program per plan, refused for rejected plans, as at
backend.py:817-846). replay_commands runs a Gemmini command stream on the
GPU; gemmini_schedules generates such streams (gen_baseline, gen_reuse_b,
gen_commands, gen_batched_reuse_b), counts them (modeled_counts,
modeled_objective, optimize) and checks them against the GEMM
(check_program).
"""
from ._locate import add_repo_to_path

add_repo_to_path()

from veritac_amd.specializations.hip_gemm.backend import (  # noqa: E402,F401
    DIM, HipGemmError, PackedB, VARIANTS, emit_c, gen_candidates, make_plan, modeled_counts,
    modeled_objective, native_check, optimize, pack_b, required_resources, run, run_flat,
    sha256_file, validate_plan)
from veritac_amd.specializations.hip_gemm.inputs import deterministic_inputs  # noqa: E402,F401
from veritac_amd.specializations.hip_gemm.replay import (  # noqa: E402,F401
    run_commands as replay_commands)
from veritac_amd.specializations.hip_gemm import schedules as gemmini_schedules  # noqa: E402,F401

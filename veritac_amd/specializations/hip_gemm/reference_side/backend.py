"""hip_gemm backend, reference side: the verbs of
specializations/gemmini_gemm/backend.py for the MI355X GEMM.

make_plan, required_resources, validate_plan, gen_candidates, modeled_counts,
modeled_objective, optimize (candidates carry check{accepted, reason}, as in
backend.py:1083-1091), and run / run_flat, which raise HipGemmError where
run_commands raises GemminiError.
"""
from ._locate import add_repo_to_path

add_repo_to_path()

from veritac_amd.specializations.hip_gemm.backend import (  # noqa: E402,F401
    DIM, HipGemmError, PackedB, VARIANTS, gen_candidates, make_plan, modeled_counts,
    modeled_objective, native_check, optimize, pack_b, required_resources, run, run_flat,
    validate_plan)
from veritac_amd.specializations.hip_gemm.inputs import deterministic_inputs  # noqa: E402,F401
from veritac_amd.specializations.hip_gemm.replay import (  # noqa: E402,F401
    run_commands as replay_commands)

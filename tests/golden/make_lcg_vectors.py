"""Record input/output vectors of the reference's deterministic_inputs.

The "lcg" mode of deterministic_inputs (specializations/gemmini_gemm/
backend.py:583-593) maps each LCG state to ((x >> 16) % 256) - 128. No
recorded reference output uses that stream (the Spike fixtures use the
two's-complement lcg8 stream of run_raw_spike.py:133-151), so nothing else
fixes the absolute values the oracle's restatement produces. This script
loads that one module from the reference checkout in THIS container (it
imports only the standard library), calls deterministic_inputs and
scalar_matmul on a few shapes, seeds and modes, and writes the results as
data to tests/golden/lcg_inputs.json. Nothing from the reference is copied or
shipped: the fixture holds numbers only.

Usage: python tests/golden/make_lcg_vectors.py [reference_root]
"""
import importlib.util
import json
import os
import sys

CASES = [  # m, n, k, seed, mode
    (2, 2, 2, 0, "lcg"), (4, 3, 5, 1, "lcg"), (16, 16, 16, 0x12345678, "lcg"),
    (3, 17, 9, 2**32 - 1, "lcg"), (32, 16, 48, 7, "lcg"), (1, 1, 1, 12345, "lcg"),
    (2, 3, 4, 9, "max"), (2, 3, 4, 9, "minmax"), (2, 3, 4, 9, "min"), (2, 3, 4, 9, "zero"),
]


def main(root="/root/reference"):
    path = os.path.join(root, "specializations", "gemmini_gemm", "backend.py")
    spec = importlib.util.spec_from_file_location("_reference_gemmini_backend", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    cases = []
    for m, n, k, seed, mode in CASES:
        A, B = mod.deterministic_inputs(m, n, k, seed, mode)
        C = mod.scalar_matmul(A, B, m, n, k)
        cases.append({"m": m, "n": n, "k": k, "seed": seed, "mode": mode,
                      "A": A, "B": B, "C": C})
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lcg_inputs.json")
    with open(out, "w") as fh:
        json.dump({"source": "specializations/gemmini_gemm/backend.py:569-602 "
                             "(deterministic_inputs, scalar_matmul), called in the build "
                             "container by tests/golden/make_lcg_vectors.py",
                   "cases": cases}, fh, separators=(",", ":"))
        fh.write("\n")
    print("wrote", out, len(cases), "cases")


if __name__ == "__main__":
    main(*sys.argv[1:])

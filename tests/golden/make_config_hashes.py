"""Full-size output hashes of the five benchmark configurations.

For each configuration (veritac_amd/specializations/hip_gemm/inputs.py
config_inputs, seed 0; configuration 4 at M = 1 and M = 16) this computes
C = D + A.B with the oracle's numpy restatement (oracle/gemm_oracle.py
gemm_i8: int64 for small shapes, exact float64 BLAS for large ones) and
records the sha256 of the row-major bytes of A, B, D and C. The GPU tests
compare the bytes vt_gemm_i8 writes with these hashes, which makes the
full-size outputs bit-exact against the oracle without shipping them.

Usage: python tests/golden/make_config_hashes.py   (about 30 s, 4 GB of memory)
"""
import hashlib
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import gemm_oracle  # noqa: E402
from veritac_amd.specializations.hip_gemm import inputs  # noqa: E402


def record(a):
    return {"dtype": str(a.dtype), "shape": list(a.shape),
            "sha256": hashlib.sha256(a.tobytes()).hexdigest()}


def main():
    cases = []
    for config, m in ((1, None), (2, None), (3, None), (4, 1), (4, 16), (5, None)):
        c = inputs.config_inputs(config, seed=0, m=m)
        C = gemm_oracle.gemm_i8(c["A"], c["B"], c["D"])
        entry = {"config": config, "m": m, "seed": 0, "A": record(c["A"]), "B": record(c["B"]),
                 "D": None if c["D"] is None else record(c["D"]), "C": record(C)}
        cases.append(entry)
        print(config, m, entry["C"]["shape"], entry["C"]["sha256"], flush=True)
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "config_hashes.json")
    with open(out, "w") as fh:
        json.dump({"generator": "inputs.config_inputs(config, seed=0, m)",
                   "oracle": "oracle.gemm_oracle.gemm_i8", "cases": cases}, fh, indent=1)
        fh.write("\n")


if __name__ == "__main__":
    main()

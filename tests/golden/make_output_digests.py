"""Extract the reference's recorded GEMM output digests into a JSON fixture.

Reads, as data only, every `local_execution.json` under
/root/reference/benchmarks/gemmini/blind_search/ together with the plan in
the run's `task.json`. Each such file records, for six deterministic input
patterns (mode, seed) of `deterministic_inputs` (specializations/
gemmini_gemm/backend.py:583-602), the sha256 of `json.dumps(C)` for the
flat int32 output list C of the run's command stream, whether C equalled the
scalar GEMM, and the interpreter's statistics
(benchmarks/gemmini/blind_search/2026-09-17/check_local_execution.py:47-53).
Nothing from the reference is imported or executed.

Usage: python tests/golden/make_output_digests.py [reference_root]
"""
import json
import os
import sys


def main(root="/root/reference"):
    base = os.path.join(root, "benchmarks", "gemmini", "blind_search")
    runs = []
    for dirpath, _, files in sorted(os.walk(base)):
        if "local_execution.json" not in files or "task.json" not in files:
            continue
        with open(os.path.join(dirpath, "local_execution.json")) as fh:
            local = json.load(fh)
        with open(os.path.join(dirpath, "task.json")) as fh:
            plan = json.load(fh)["plan"]
        runs.append({
            "name": os.path.relpath(dirpath, base).replace(os.sep, "/"),
            "plan": plan,
            "success": local["success"],
            "cases": [{"mode": c["mode"], "seed": c["seed"],
                       "all_outputs_match": c["all_outputs_match"],
                       "output_sha256": c["output_sha256"], "stats": c["stats"]}
                      for c in local["cases"]],
        })
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "output_digests.json")
    with open(out, "w") as fh:
        json.dump({"source": "benchmarks/gemmini/blind_search/*/local_execution.json",
                   "digest": "sha256(json.dumps(C).encode()), C the flat int32 output list",
                   "runs": runs}, fh, indent=1)
        fh.write("\n")
    print("%d runs, %d cases -> %s" % (len(runs), sum(len(r["cases"]) for r in runs), out))


if __name__ == "__main__":
    main(*sys.argv[1:])

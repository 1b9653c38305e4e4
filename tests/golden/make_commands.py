"""Extract the reference's Gemmini command streams into a JSON fixture.

Reads, as data only, every `request.json` under
/root/reference/benchmarks/gemmini/ and keeps its `plan` and `commands`
fields (schema veritac_program_request_v1, specializations/gemmini_gemm/
backend.py:891-936); the `encoding` field is never read. For the four
blind-search rejection witnesses it also keeps, from `result.json`, the
recorded counterexample: the sparse input (`sparse_inputs`: flat indices of A
and B set to one, everything else zero) and the output cell that differs
from A.B (`row`, `col`, `actual`, `expected`). Streams whose plan and
per-run command counts match a recorded Spike run
(benchmarks/gemmini/results/raw_*/report.json `plan` and `executed_commands`)
are linked to that run, whose COUT outputs tests/golden/spike_cout.json holds.
Nothing from the reference is imported or executed.

Usage: python tests/golden/make_commands.py [reference_root]
"""
import json
import os
import sys


def counts(commands):
    out = {}
    for c in commands:
        out[c["kind"]] = out.get(c["kind"], 0) + 1
    return out


def main(root="/root/reference"):
    base = os.path.join(root, "benchmarks", "gemmini")
    runs = {}
    results = os.path.join(base, "results")
    for name in sorted(os.listdir(results)):
        rep = os.path.join(results, name, "report.json")
        if name.startswith("raw_") and os.path.exists(rep):
            with open(rep) as fh:
                report = json.load(fh)
            ops = report["executed_commands"]["operations"]
            modes = len(report["output_checks"]["modes"])
            per_run = {k: ops[k] // modes for k in ("mvin", "preload", "compute", "mvout")}
            runs[name] = (report["plan"], per_run)
    streams = []
    for dirpath, _, files in sorted(os.walk(base)):
        if "request.json" not in files:
            continue
        with open(os.path.join(dirpath, "request.json")) as fh:
            req = json.load(fh)
        rel = os.path.relpath(dirpath, base)
        entry = {"name": rel.replace(os.sep, "/"),
                 "source": "benchmarks/gemmini/%s/request.json" % rel.replace(os.sep, "/"),
                 "plan": req["plan"], "commands": req["commands"]}
        c = counts(req["commands"])
        for run, (plan, per_run) in runs.items():
            if plan == req["plan"] and all(c.get(k, 0) == v for k, v in per_run.items()):
                entry["spike_run"] = run
        res = os.path.join(dirpath, "result.json")
        if "rejection_witnesses" in rel and os.path.exists(res):
            with open(res) as fh:
                w = json.load(fh)["witness"]
            entry["witness"] = {k: w[k] for k in ("sparse_inputs", "row", "col", "actual", "expected")}
        streams.append(entry)
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemmini_commands.json")
    with open(out, "w") as fh:
        json.dump({"format": "plan + commands of veritac_program_request_v1 requests",
                   "streams": streams}, fh, indent=None, separators=(",", ":"))
        fh.write("\n")
    linked = sum("spike_run" in s for s in streams)
    print("wrote %d streams (%d linked to Spike runs, %d witnesses) to %s"
          % (len(streams), linked, sum("witness" in s for s in streams), out))


if __name__ == "__main__":
    main(*sys.argv[1:])

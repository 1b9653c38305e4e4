"""Extract the reference's recorded Spike GEMM outputs into a JSON fixture.

Reads, as data only, the 8 run directories
/root/reference/benchmarks/gemmini/results/raw_*/ : `report.json` (only its
`plan` and `sizes` fields) and `raw_spike_outputs.txt` (lines
"COUT <mode-index> <%08x per int32>", format of
specializations/gemmini_gemm/runtime/run_raw_spike.py:409-423, mode order
zeros/extrema/lcg from run_raw_spike.py:26). Nothing from the reference is
imported or executed. Output: tests/golden/spike_cout.json with one entry per
run: name, plan (m, n, k, schedule), sizes, and for each mode the int32
outputs as a hex string (8 hex digits per value, as recorded).

Usage: python tests/golden/make_golden.py [reference_root]
"""
import json
import os
import re
import sys

MODES = ("zeros", "extrema", "lcg")
COUT = re.compile(r"^COUT (\d+) ([0-9a-f]+)$")


def main(root="/root/reference"):
    base = os.path.join(root, "benchmarks", "gemmini", "results")
    runs = []
    for name in sorted(os.listdir(base)):
        d = os.path.join(base, name)
        if not (name.startswith("raw_") and os.path.isdir(d)):
            continue
        with open(os.path.join(d, "report.json")) as fh:
            report = json.load(fh)
        plan = report["plan"]
        outputs = {}
        with open(os.path.join(d, "raw_spike_outputs.txt")) as fh:
            for line in fh:
                m = COUT.match(line.strip())
                if m:
                    outputs[MODES[int(m.group(1))]] = m.group(2)
        assert set(outputs) == set(MODES), (name, sorted(outputs))
        for mode, hx in outputs.items():
            assert len(hx) == 8 * plan["m"] * plan["n"], (name, mode)
        runs.append({
            "name": name,
            "source": "benchmarks/gemmini/results/%s/raw_spike_outputs.txt" % name,
            "plan": {k: plan[k] for k in ("m", "n", "k", "schedule")},
            "sizes": report["sizes"],
            "cout": outputs,
        })
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "spike_cout.json")
    with open(out, "w") as fh:
        json.dump({"format": "int32 outputs, 8 hex digits each, row-major m x n",
                   "modes": list(MODES), "runs": runs}, fh, indent=1)
    print("wrote %d runs (%d vectors) to %s" % (len(runs), 3 * len(runs), out))


if __name__ == "__main__":
    main(*sys.argv[1:])

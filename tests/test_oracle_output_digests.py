"""Pin the oracle, the deterministic input generator and the report's list
digest against the reference's recorded output hashes.

tests/golden/output_digests.json holds, for the eight blind-search runs
with a local execution record (benchmarks/gemmini/blind_search/2026-09-17/
{runs,compact_runs}/*/local_execution.json), six (mode, seed) input
patterns each, the sha256 of json.dumps of the flat output list, and the
interpreter statistics of the run's certified command stream
(check_local_execution.py:47-53). 48 recorded hashes fix the scalar GEMM of
deterministic_inputs bit for bit; the statistics fix the command counting of
the oracle's interpreter.
"""
import numpy as np
import pytest

from conftest import winner_stream
from oracle import gemm_oracle, gemmini_replay
from veritac_amd.specializations.hip_gemm import inputs, provenance


def _cases(runs):
    return [(r, c) for r in runs for c in r["cases"]]


def test_fixture_shape(output_digests):
    assert len(output_digests) == 8
    assert all(len(r["cases"]) == 6 and r["success"] for r in output_digests)
    assert {(c["mode"], c["seed"]) for r in output_digests for c in r["cases"]} == \
        {("zero", 0), ("max", 0), ("min", 0), ("minmax", 0), ("lcg", 0), ("lcg", 917)}


def test_scalar_gemm_reproduces_recorded_hashes(output_digests):
    for run, case in _cases(output_digests):
        p = run["plan"]
        a, b = gemm_oracle.deterministic_inputs(p["m"], p["n"], p["k"], case["seed"], case["mode"])
        c = gemm_oracle.scalar_matmul(a, b, p["m"], p["n"], p["k"])
        assert provenance.list_digest(c) == case["output_sha256"], (run["name"], case)


def test_replay_reproduces_recorded_hashes_and_stats(output_digests, commands):
    for run, case in _cases(output_digests):
        p = run["plan"]
        stream = winner_stream(commands, run["name"])
        a, b = gemm_oracle.deterministic_inputs(p["m"], p["n"], p["k"], case["seed"], case["mode"])
        c, stats = gemmini_replay.run_commands(stream["commands"], stream["plan"], a, b)
        assert stats == case["stats"], run["name"]
        assert provenance.list_digest(c) == case["output_sha256"], (run["name"], case)


def test_numpy_inputs_match_the_scalar_generator(output_digests):
    for run, case in _cases(output_digests):
        p = run["plan"]
        a, b = gemm_oracle.deterministic_inputs(p["m"], p["n"], p["k"], case["seed"], case["mode"])
        na, nb = inputs.deterministic_inputs(p["m"], p["n"], p["k"], case["seed"], case["mode"])
        assert na.reshape(-1).tolist() == a and nb.reshape(-1).tolist() == b


def test_planted_error_changes_the_hash(output_digests):
    """A one-off output element, a transposed output and a dropped k term all
    miss every recorded hash of their case."""
    run = output_digests[0]
    p = run["plan"]
    case = next(c for c in run["cases"] if c["mode"] == "lcg")
    a, b = gemm_oracle.deterministic_inputs(p["m"], p["n"], p["k"], case["seed"], "lcg")
    c = gemm_oracle.scalar_matmul(a, b, p["m"], p["n"], p["k"])
    bumped = list(c)
    bumped[7] += 1
    assert provenance.list_digest(bumped) != case["output_sha256"]
    ct = np.array(c).reshape(p["m"], p["n"]).T.reshape(-1).tolist()
    assert provenance.list_digest(ct) != case["output_sha256"]
    A = np.array(a, dtype=np.int64).reshape(p["m"], p["k"])
    B = np.array(b, dtype=np.int64).reshape(p["k"], p["n"])
    short = (A[:, 1:] @ B[1:, :]).reshape(-1).tolist()
    assert provenance.list_digest(short) != case["output_sha256"]

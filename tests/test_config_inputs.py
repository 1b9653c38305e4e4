"""The benchmark configurations' inputs are reproducible: the seeded
generator still produces the operands whose oracle outputs
tests/golden/config_hashes.json records (so the GPU tests that compare
full-size outputs with those hashes compare against the right inputs)."""
import hashlib
import json
import os

import pytest

from veritac_amd.specializations.hip_gemm import inputs

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
with open(os.path.join(ROOT, "tests", "golden", "config_hashes.json")) as fh:
    CASES = json.load(fh)["cases"]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "config%d_m%s" % (c["config"], c["m"]))
def test_config_inputs_match_recorded_hashes(case):
    c = inputs.config_inputs(case["config"], seed=case["seed"], m=case["m"])
    for name in ("A", "B", "D"):
        rec = case[name]
        if rec is None:
            assert c[name] is None
            continue
        a = c[name]
        assert [str(a.dtype), list(a.shape)] == [rec["dtype"], rec["shape"]]
        assert hashlib.sha256(a.tobytes()).hexdigest() == rec["sha256"], name
    batch, M, N, K, has_d, b_shared = inputs.config_shape(case["config"], case["m"])
    assert case["C"]["shape"] == ([batch, M, N] if batch > 1 else [M, N])

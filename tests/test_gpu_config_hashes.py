"""Full-size outputs of the five benchmark configurations, bit-exact against
the oracle: the sha256 of the bytes vt_gemm_i8 writes must equal the hash
of the oracle's output recorded in tests/golden/config_hashes.json, for
every kernel variant that accepts the shape."""
import hashlib
import json
import os

import pytest

torch = pytest.importorskip("torch")

from veritac_amd import _lib
from veritac_amd.specializations.hip_gemm import backend as hg
from veritac_amd.specializations.hip_gemm import inputs

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
with open(os.path.join(ROOT, "tests", "golden", "config_hashes.json")) as fh:
    CASES = json.load(fh)["cases"]


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    assert _lib.load_library().vt_device_count() >= 1, "GPU visible but not gfx950"
    return torch.device("cuda", 0)


def variants(M):
    out = ["auto", "generic", "mfma_256x256", "mfma_256x128", "mfma_128x128"]
    if M <= hg.SKINNY_MAX_M:
        out.append("skinny")
    return out


@pytest.mark.parametrize("case", CASES, ids=lambda c: "config%d_m%s" % (c["config"], c["m"]))
def test_full_size_output_matches_oracle_hash(dev, case):
    c = inputs.config_inputs(case["config"], seed=case["seed"], m=case["m"])
    batch, M, N, K, has_d, b_shared = inputs.config_shape(case["config"], case["m"])
    A = torch.from_numpy(c["A"]).to(dev)
    B = torch.from_numpy(c["B"]).to(dev)
    D = None if c["D"] is None else torch.from_numpy(c["D"]).to(dev)
    dmax = 0 if D is None else int(D.abs().max())
    for variant in variants(M):
        print("config", case["config"], "m", case["m"], variant, flush=True)
        plan = hg.make_plan(M, N, K, batch=batch, b_shared=b_shared, has_d=has_d,
                            d_max_abs=dmax, variant=variant)
        C = hg.run(plan, A, B, D)
        torch.cuda.synchronize(dev)
        got = hashlib.sha256(C.cpu().numpy().tobytes()).hexdigest()
        assert got == case["C"]["sha256"], (case["config"], case["m"], variant)
        del C

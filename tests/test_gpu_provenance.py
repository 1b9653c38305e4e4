"""Device profile, recorded output hashes and run reports on the GPU.

* probe() on the MI355X returns a valid "hip" profile of a gfx950 device;
* vt_gemm_i8 (every applicable variant) and the command-stream replay
  reproduce the 48 output hashes the reference recorded for its
  blind-search runs (tests/golden/output_digests.json), and the replay
  reproduces the recorded interpreter statistics;
* run_report binds the hashes to the bytes it checked, reports a planted
  wrong result as a failure, and carries timings when asked.
"""
import hashlib
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from conftest import winner_stream
from oracle import gemm_oracle as go
from veritac_amd import _lib
from veritac_amd.specializations.hip_gemm import backend as hg
from veritac_amd.specializations.hip_gemm import inputs, provenance
from veritac_amd.specializations.hip_gemm import replay as rp

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    assert _lib.load_library().vt_device_count() >= 1, "GPU visible but not gfx950"
    return torch.device("cuda", 0)


def say(*args):
    print(*args, flush=True)


def test_probe_describes_the_gfx950_device(dev):
    p = provenance.probe()
    assert p is not None
    say("profile", provenance.canonical_json(p))
    provenance.validate_schema(p)
    assert p["backend"] == "hip" and p["gcn_arch_name"].split(":")[0] == "gfx950"
    assert p["simd_width"] == 64 and p["compute_units"] == torch.cuda.get_device_properties(
        dev).multi_processor_count
    assert p["max_threadgroup_memory_bytes"] >= 64 * 1024
    assert p["toolchain"]["code_target"] == "gfx950"
    assert p["toolchain"]["version"] != "unknown"
    assert all(provenance.feature_authorized(p, f) for f in provenance.GFX950_FEATURES)
    assert provenance.profile_hash(p) == provenance.profile_hash(provenance.probe())


def _variants(plan):
    out = ["auto", "generic"]
    if plan["n"] % 16 == 0 and plan["k"] % 16 == 0:
        out += ["mfma_256x256", "mfma_256x128", "mfma_128x128"]
        if plan["m"] <= hg.SKINNY_MAX_M:
            out.append("skinny")
    return out


def test_gemm_reproduces_the_recorded_output_hashes(dev, output_digests):
    for run in output_digests:
        p = run["plan"]
        for case in run["cases"]:
            a, b = inputs.deterministic_inputs(p["m"], p["n"], p["k"], case["seed"], case["mode"])
            A = torch.from_numpy(a).to(dev)
            B = torch.from_numpy(b).to(dev)
            for variant in _variants(p):
                say("gemm", run["name"], case["mode"], case["seed"], variant)
                plan = hg.make_plan(p["m"], p["n"], p["k"], variant=variant)
                C = hg.run(plan, A, B)
                torch.cuda.synchronize(dev)
                got = provenance.list_digest(C.cpu().reshape(-1).tolist())
                assert got == case["output_sha256"], (run["name"], case["mode"], variant)


def test_replay_reproduces_the_recorded_hashes_and_stats(dev, output_digests, commands):
    for run in output_digests:
        p = run["plan"]
        stream = winner_stream(commands, run["name"])
        for case in run["cases"]:
            say("replay", run["name"], case["mode"], case["seed"])
            a, b = go.deterministic_inputs(p["m"], p["n"], p["k"], case["seed"], case["mode"])
            C, stats = rp.run_commands(stream["commands"], stream["plan"], a, b, device=dev)
            assert stats == case["stats"], run["name"]
            assert provenance.list_digest(C) == case["output_sha256"], (run["name"], case)


def test_run_report_binds_the_checked_bytes(dev, tmp_path):
    plan = hg.make_plan(256, 384, 512)
    say("report", plan["variant"])
    rep = provenance.run_report(plan, mode="lcg", seed=917, out_dir=str(tmp_path))
    assert rep["success"] and rep["verification"]["passed"]
    a, b = inputs.deterministic_inputs(256, 384, 512, 917, "lcg")
    expect = go.gemm_i8_int64(a, b).astype(np.int32)
    assert rep["output"]["sha256"] == hashlib.sha256(expect.tobytes()).hexdigest()
    assert rep["output_list_sha256"] == provenance.list_digest(expect.reshape(-1).tolist())
    assert rep["operands"]["A"]["sha256"] == hashlib.sha256(a.tobytes()).hexdigest()
    assert rep["operands"]["B"]["sha256"] == hashlib.sha256(b.tobytes()).hexdigest()
    assert rep["device_profile_sha256"] == provenance.profile_hash(provenance.probe())
    lib = rep["artifacts"]["library"]
    assert lib["sha256"] == provenance.sha256_file(_lib.library_path())
    body = {k: v for k, v in rep.items() if k != "report_sha256"}
    assert rep["report_sha256"] == provenance.digest(body)
    assert os.path.isfile(tmp_path / "report.json")


def test_report_of_a_wrong_result_fails(dev):
    plan = hg.make_plan(512, 512, 1024)
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    A = torch.randint(-128, 128, (512, 1024), dtype=torch.int8, device=dev, generator=g)
    B = torch.randint(-128, 128, (1024, 512), dtype=torch.int8, device=dev, generator=g)
    C = hg.run(plan, A, B)
    torch.cuda.synchronize(dev)
    good = provenance.report_from_result(plan, A, B, None, C)
    assert good["success"]
    C[100, 200] += 1
    C[300, 7] -= 1
    bad = provenance.report_from_result(plan, A, B, None, C)
    assert not bad["success"] and bad["output"]["sha256"] != good["output"]["sha256"]


def test_run_report_with_d_batch_and_timing(dev):
    plan = hg.make_plan(64, 256, 512, batch=4, has_d=True, d_max_abs=1 << 20)
    rep = provenance.run_report(plan, seed=5, benchmark_runs=5)
    assert rep["success"] and "D" in rep["operands"]
    assert rep["timing"]["num_runs"] == 5 and rep["timing"]["gpu_time_ms"] > 0
    assert "output_list_sha256" not in rep        # batched: raw-byte hash only

"""Host-side tests of the hardware profile, the report hashes and the exact
result check (specializations/hip_gemm/provenance.py and verify.py).

The profile tests follow the reference's tests/test_hardware_profile.py
(schema acceptance and rejection, canonical JSON, hashing, rendering,
save / load, feature authorisation) for the "hip" backend. The exact check
runs here on CPU tensors, with results computed by numpy's int64 matmul and
mistakes planted in them.
"""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

from veritac_amd import _lib
from veritac_amd.specializations.hip_gemm import backend, provenance, verify


def valid():
    return provenance.make_hip_profile()


# --- schema ---------------------------------------------------------------

def test_accepts_valid():
    provenance.validate_schema(valid())


@pytest.mark.parametrize("bad", [None, [], "profile", 3])
def test_rejects_non_dict(bad):
    with pytest.raises(ValueError):
        provenance.validate_schema(bad)


@pytest.mark.parametrize("field,value", [
    ("schema_version", 2), ("schema_version", None),
    ("backend", "rocm"), ("backend", None),
    ("device_name", ""), ("device_name", "  "), ("device_name", 7),
    ("max_threads_per_threadgroup", 0), ("max_threads_per_threadgroup", True),
    ("max_threadgroup_memory_bytes", -1), ("max_threadgroup_memory_bytes", 1.5),
    ("simd_width", None), ("simd_width", False),
    ("toolchain", None), ("toolchain", {"name": "hip_runtime"}),
    ("toolchain", {"name": "", "version": "7.0"}),
    ("provenance", {"source": "hip_device_query"}), ("provenance", "x"),
    ("features", None), ("features", {"matrix_ops": 1}), ("features", {"x": "yes"}),
])
def test_rejects_malformed(field, value):
    p = valid()
    p[field] = value
    with pytest.raises(ValueError):
        provenance.validate_schema(p)


def test_accepts_bool_and_none_features():
    p = valid()
    p["features"] = {"a": True, "b": False, "c": None}
    provenance.validate_schema(p)


def test_canonical_json_is_sorted_compact_and_validated():
    p = valid()
    text = provenance.canonical_json(p)
    assert text == json.dumps(json.loads(text), sort_keys=True, separators=(",", ":"))
    shuffled = dict(reversed(list(p.items())))
    assert provenance.canonical_json(shuffled) == text
    assert provenance.profile_hash(shuffled) == hashlib.sha256(text.encode()).hexdigest()
    bad = dict(p, simd_width=0)
    with pytest.raises(ValueError):
        provenance.canonical_json(bad)
    with pytest.raises(ValueError):
        provenance.profile_hash(bad)
    assert provenance.canonical_json(bad, validate=False)


def test_hash_changes_with_any_field():
    base = provenance.profile_hash(valid())
    assert provenance.profile_hash(provenance.make_hip_profile(compute_units=255)) != base
    assert provenance.profile_hash(provenance.make_hip_profile(host="other")) != base


def test_render_marks_unknown_and_validates():
    p = provenance.make_hip_profile(supported=False, arch="gfx942")
    text = provenance.render_prompt(p)
    assert text.startswith("[hardware_profile]\n")
    assert "backend: hip" in text and "simd_width: 64" in text
    assert "matrix_ops: unknown (cannot authorize)" in text
    assert "toolchain: hip_runtime 7.0.51831" in text
    with pytest.raises(ValueError):
        provenance.render_prompt(dict(p, backend="x"))


def test_save_and_load_roundtrip(tmp_path):
    p = valid()
    path = str(tmp_path / "profile.json")
    h = provenance.save(p, path)
    assert h == provenance.profile_hash(p)
    assert provenance.load(path) == p
    with open(path, "w") as fh:
        json.dump(dict(p, schema_version=9), fh)
    with pytest.raises(ValueError):
        provenance.load(path)
    with pytest.raises(ValueError):
        provenance.save(dict(p, backend=None), str(tmp_path / "bad.json"))


def test_feature_authorisation():
    p = valid()
    assert provenance.feature_authorized(p, "matrix_ops")
    assert provenance.feature_authorized(p, "sramecc")
    assert not provenance.feature_authorized(p, "xnack")          # explicit False
    assert not provenance.feature_authorized(p, "not_a_feature")  # absent
    unknown = provenance.make_hip_profile(supported=False, arch="gfx942")
    assert not any(provenance.feature_authorized(unknown, f)
                   for f in provenance.GFX950_FEATURES)
    with pytest.raises(ValueError):
        provenance.feature_authorized(dict(p, features=[]), "matrix_ops")


def test_normalisation_of_the_device_query():
    p = provenance.make_hip_profile()
    assert p["backend"] == "hip" and p["simd_width"] == 64
    assert p["max_threadgroup_memory_bytes"] == 160 * 1024
    assert p["toolchain"]["code_target"] == "gfx950"
    assert p["features"]["xnack"] is False and p["features"]["sramecc"] is True
    assert provenance.make_hip_profile(arch="gfx950")["features"]["xnack"] is None
    assert p["device_name_source"] == "hip_runtime"
    blank = provenance.make_hip_profile(device_name="")
    assert blank["device_name"] == "AMD gfx950 (256 CUs)"
    assert blank["device_name_source"] == "gcn_arch_name"
    provenance.validate_schema(blank)
    assert provenance.hip_version_string(70051831) == "7.0.51831"
    assert provenance.hip_version_string(60443483) == "6.4.43483"
    assert provenance.hip_version_string(0) == "unknown"


def test_probe_returns_none_without_a_device():
    if torch.cuda.is_available():
        pytest.skip("a HIP device is present")
    assert provenance.probe() is None


def test_probe_returns_none_without_the_library(monkeypatch):
    def refuse(device=-1):
        raise _lib.HipGemmError("library missing", _lib.VT_ENODEV)
    monkeypatch.setattr(_lib, "device_query", refuse)
    assert provenance.probe() is None


def test_probe_normalises_the_query(monkeypatch):
    raw = {"name": "AMD Instinct MI355X", "arch": "gfx950:sramecc+:xnack-",
           "code_object_arch": "gfx950", "total_memory_bytes": 309_220_868_096,
           "l2_cache_bytes": 4194304, "lds_per_workgroup_bytes": 163840,
           "lds_per_cu_bytes": 163840, "compute_units": 256, "wavefront_size": 64,
           "max_threads_per_workgroup": 1024, "max_clock_khz": 2400000,
           "memory_clock_khz": 2000000, "memory_bus_width_bits": 8192, "pci_domain": 0,
           "pci_bus": 5, "pci_device": 0, "hip_runtime_version": 70051831,
           "hip_driver_version": 70051831, "supported": 1}
    monkeypatch.setattr(_lib, "device_query", lambda device=-1: dict(raw))
    p = provenance.probe()
    assert p["compute_units"] == 256 and p["pci"]["bus"] == 5
    assert provenance.feature_authorized(p, "int8_matrix_ops")
    monkeypatch.setattr(_lib, "device_query", lambda device=-1: dict(raw, wavefront_size=0))
    assert provenance.probe() is None     # a profile that fails validation is not returned


# --- hashes ---------------------------------------------------------------

def test_digest_formats():
    plan = {"m": 16, "n": 16, "k": 16}
    assert provenance.digest(plan) == hashlib.sha256(b'{"k":16,"m":16,"n":16}').hexdigest()
    assert provenance.list_digest([1, -2, 3]) == hashlib.sha256(b"[1, -2, 3]").hexdigest()


def test_array_record_is_layout_exact():
    a = np.arange(12, dtype=np.int32).reshape(3, 4)
    rec = provenance.array_record(a)
    assert rec == {"dtype": "int32", "shape": [3, 4],
                   "sha256": hashlib.sha256(a.tobytes()).hexdigest()}
    assert provenance.array_record(torch.from_numpy(a)) == rec
    assert provenance.array_record(a.T)["sha256"] != rec["sha256"]          # row-major bytes
    assert provenance.array_record(a.astype(">i4")) == rec                  # little-endian
    assert provenance.array_record(a.astype(np.int64))["sha256"] != rec["sha256"]


def test_artifact_hashes_cover_library_sources_and_modules():
    arts = provenance.artifact_hashes()
    for name in ("library", "header", "binding", "build_recipe", "hip_source:vt_hip_gemm.hip",
                 "module:backend", "module:verify", "module:replay", "module:provenance"):
        assert name in arts, name
    src = arts["hip_source:vt_hip_gemm.hip"]
    assert src["path"] == "veritac_amd/csrc/vt_hip_gemm.hip"
    assert src["sha256"] == provenance.sha256_file(os.path.join(provenance.ROOT, src["path"]))


# --- exact check ----------------------------------------------------------

def _case(m, n, k, batch=None, shared=False, with_d=False, seed=0):
    rng = np.random.default_rng(seed)
    lead = () if batch is None else (batch,)
    A = rng.integers(-128, 128, lead + (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, ((k, n) if (batch is None or shared) else lead + (k, n)),
                     dtype=np.int8)
    D = rng.integers(-2**20, 2**20, lead + (m, n), dtype=np.int32) if with_d else None
    C = np.matmul(A.astype(np.int64), B.astype(np.int64))
    if D is not None:
        C = C + D
    t = [torch.from_numpy(x) if x is not None else None for x in (A, B, D)]
    return t[0], t[1], t[2], torch.from_numpy(C.astype(np.int32))


@pytest.mark.parametrize("kw", [dict(m=33, n=48, k=80), dict(m=16, n=64, k=256, with_d=True),
                                dict(m=8, n=16, k=32, batch=3),
                                dict(m=8, n=16, k=32, batch=3, shared=True, with_d=True)])
def test_exact_check_accepts_correct_results(kw):
    A, B, D, C = _case(**kw)
    r = verify.exact_check(A, B, C, D)
    assert r["passed"] and r["projections_equal"] and r["checksums_equal"]
    assert r["miss_probability_bound"] == 2.0 ** -16


@pytest.mark.parametrize("delta", [1, -1, 2**31, 12345, 2**16])
def test_exact_check_rejects_a_single_wrong_element(delta):
    A, B, D, C = _case(40, 32, 64, with_d=True)
    for pos in ((0, 0), (39, 31), (17, 5)):
        bad = C.clone()
        bad[pos] = int((np.int64(bad[pos]) + delta + 2**31) % 2**32 - 2**31)
        r = verify.exact_check(A, B, bad, D)
        assert not r["passed"] and not r["checksums_equal"], (delta, pos)


def test_exact_check_rejects_cancelling_and_structural_mistakes():
    A, B, D, C = _case(32, 32, 64)
    swap = C.clone()              # a 2x2 pattern of +e / -e leaves every row and column sum
    swap[3, 4] += 7
    swap[3, 9] -= 7
    swap[20, 4] -= 7
    swap[20, 9] += 7
    r = verify.exact_check(A, B, swap, None)
    assert r["checksums_equal"] and not r["projections_equal"] and not r["passed"]
    assert not verify.exact_check(A, B, C.T.contiguous(), None)["passed"]
    assert not verify.exact_check(A, B, C, torch.ones_like(C))["passed"]   # D ignored
    short = torch.from_numpy((A.numpy()[:, 1:].astype(np.int64) @
                              B.numpy()[1:].astype(np.int64)).astype(np.int32))
    assert not verify.exact_check(A, B, short, None)["passed"]             # dropped k term


def test_exact_check_accepts_the_wrapped_int32_sum():
    """Outside the legality bound the contract is the product modulo 2^32."""
    A = torch.full((4, 8192), -128, dtype=torch.int8)
    B = torch.full((8192, 4), -128, dtype=torch.int8)
    true = 8192 * 128 * 128                  # 2^27: no wrap
    D = torch.full((4, 4), 2**31 - 1, dtype=torch.int32)
    wrapped = (true + 2**31 - 1 + 2**31) % 2**32 - 2**31
    C = torch.full((4, 4), wrapped, dtype=torch.int32)
    assert verify.exact_check(A, B, C, D)["passed"]
    C2 = C.clone()
    C2[0, 0] = 2**31 - 1                   # saturated instead of wrapped
    assert not verify.exact_check(A, B, C2, D)["passed"]


def test_exact_check_refuses_inconsistent_shapes_and_inexact_sizes():
    A, B, D, C = _case(8, 16, 32)
    with pytest.raises(verify.VerifyError):
        verify.exact_check(A, B, C[:, :8], None)
    with pytest.raises(verify.VerifyError):
        verify.exact_check(A, B[:16], C, None)
    with pytest.raises(verify.VerifyError):
        verify.exact_check(A, B, C, D if D is not None else C[:4])
    assert verify.exactness_bound(8192, 8192, 8192) < verify.EXACT_LIMIT
    assert verify.exactness_bound(1 << 20, 1 << 20, 1 << 20) >= verify.EXACT_LIMIT


def test_report_from_result_on_host_tensors(monkeypatch):
    """The report machinery on CPU tensors with an injected profile: the
    hashes name the bytes checked, and a wrong result is reported as such."""
    plan = backend.make_plan(32, 48, 64, variant="generic")
    A, B, _, C = _case(32, 48, 64)
    prof = provenance.make_hip_profile()
    rep = provenance.report_from_result(plan, A, B, None, C, profile=prof)
    assert rep["success"] and rep["schema_version"] == 1 and rep["backend"] == "hip_gemm"
    assert rep["plan_sha256"] == provenance.digest(plan)
    assert rep["device_profile_sha256"] == provenance.profile_hash(prof)
    assert rep["output"]["sha256"] == hashlib.sha256(C.numpy().tobytes()).hexdigest()
    assert rep["output_list_sha256"] == provenance.list_digest(C.reshape(-1).tolist())
    assert rep["operands"]["A"]["sha256"] == hashlib.sha256(A.numpy().tobytes()).hexdigest()
    body = {k: v for k, v in rep.items() if k != "report_sha256"}
    assert rep["report_sha256"] == provenance.digest(body)
    json.dumps(rep)
    bad = C.clone()
    bad[1, 2] += 1
    rep2 = provenance.report_from_result(plan, A, B, None, bad, profile=prof)
    assert not rep2["success"] and rep2["output"]["sha256"] != rep["output"]["sha256"]
    with pytest.raises(_lib.HipGemmError):
        provenance.report_from_result(dict(plan, m=-1), A, B, None, C, profile=prof)

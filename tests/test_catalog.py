"""The specialization catalog (mirrors the reference's tests/test_specializations.py:15-24)."""
import json
import os
import shutil
import subprocess
import sys

import pytest

from veritac_amd.specializations import catalog

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SHIM = os.path.join(ROOT, "veritac_amd", "specializations", "hip_gemm", "reference_side")
SHIM_PREFIX = "specializations/hip_gemm/"
REFERENCE = "/root/reference"


def test_listing_imports_only_the_standard_library():
    code = ("import sys, json; from veritac_amd.specializations.catalog import list_specializations;"
            "r = list_specializations();"
            "print(json.dumps([x['id'] for x in r]));"
            "print(json.dumps(sorted(m for m in ('torch','numpy','ctypes') if m in sys.modules)))")
    out = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True,
                         check=True).stdout.splitlines()
    assert json.loads(out[0]) == ["hip_gemm"]
    assert json.loads(out[1]) == []


def test_descriptor_schema_and_paths():
    """The reference's rule (tests/test_specializations.py:19-24) on the repo's
    own descriptor: proof_scope and boundaries are non-empty, and every path
    of every list resolves under the repo root (the library once built)."""
    d = catalog.describe("hip_gemm")
    assert d["schema_version"] == 1 and d["id"] == "hip_gemm"
    for key in ("status", "computation", "target", "implementation", "formal_sources",
                "entrypoints", "proof_scope", "boundaries", "evidence"):
        assert key in d, key
    assert d["proof_scope"] and d["boundaries"]
    for path in catalog.descriptor_paths(d):
        if path.endswith(".so"):
            # a build artefact: its recipe must exist
            assert os.path.exists(os.path.join(ROOT, "veritac_amd", "build.py"))
            continue
        assert os.path.exists(os.path.join(ROOT, path)), path


def _reference_tree(tmp_path):
    """A reference tree after the maintainer's install step: the reference-side
    files copied to specializations/hip_gemm/, and the reference's own files the
    descriptor names present (placeholders here; they are checked against a
    real reference checkout separately when one is present)."""
    desc = json.load(open(os.path.join(SHIM, "specialization.json")))
    root = tmp_path / "reference"
    dst = root / "specializations" / "hip_gemm"
    shutil.copytree(SHIM, dst)
    for path in catalog.descriptor_paths(desc):
        if path.startswith(SHIM_PREFIX):
            continue
        target = root / path
        target.parent.mkdir(parents=True, exist_ok=True)
        if "." in os.path.basename(path):
            target.write_text("")
        else:
            target.mkdir(exist_ok=True)
    return root, desc


def test_reference_side_descriptor_passes_the_reference_path_rule(tmp_path):
    root, desc = _reference_tree(tmp_path)
    got = catalog.describe("hip_gemm", packages=str(root / "specializations"))
    assert got == desc
    assert got["proof_scope"] and got["boundaries"]
    for path in catalog.descriptor_paths(got):
        assert (root / path).exists(), path
    # every shipped file the descriptor names under specializations/hip_gemm/ is ours
    shipped = [p for p in catalog.descriptor_paths(got) if p.startswith(SHIM_PREFIX)]
    assert shipped and all(os.path.exists(os.path.join(SHIM, p[len(SHIM_PREFIX):]))
                           for p in shipped)


@pytest.mark.skipif(not os.path.isdir(REFERENCE), reason="no reference checkout here")
def test_reference_side_paths_exist_in_the_reference_checkout():
    """The descriptor's paths outside specializations/hip_gemm/ are the
    reference's own files (Lean contract, recorded results)."""
    desc = json.load(open(os.path.join(SHIM, "specialization.json")))
    for path in catalog.descriptor_paths(desc):
        if not path.startswith(SHIM_PREFIX):
            assert os.path.exists(os.path.join(REFERENCE, path)), path


def _run_in_tree(root, code, env_repo):
    env = dict(os.environ)
    env.pop("VT_HIP_GEMM_REPO", None)
    if env_repo is not None:
        env["VT_HIP_GEMM_REPO"] = env_repo
    return subprocess.run([sys.executable, "-c", code], cwd=str(root), capture_output=True,
                          text=True, env=env)


# The candidate loop of the reference's examples/gemmini_gemm_demo.py:41-44,
# unchanged, against hip_gemm.
DEMO_LOOP = """
import json
from specializations.hip_gemm import backend as g
search = g.optimize(%d, %d, %d)
eligible = []
for entry in search["candidates"]:
    if not entry["valid"] or not entry["check"]["accepted"]:
        continue
    eligible.append(entry["plan"]["variant"])
print(json.dumps({"keys": sorted(search["candidates"][0]), "eligible": eligible,
                  "winner": search["winner"]["variant"] if search["winner"] else None,
                  "reasons": [c["check"]["reason"] for c in search["candidates"]]}))
"""


def test_reference_style_candidate_loop_runs_unchanged(tmp_path):
    root, _ = _reference_tree(tmp_path)
    (root / "specializations" / "__init__.py").write_text("")
    proc = _run_in_tree(root, DEMO_LOOP % (8192, 8192, 8192), ROOT)
    assert proc.returncode == 0, proc.stderr
    out = json.loads(proc.stdout)
    # the keys the reference's optimize returns per candidate (backend.py:1083-1085)
    assert {"plan", "valid", "invalid_reason", "check", "counts", "objective"} <= set(out["keys"])
    assert out["winner"] == "mfma_256x256"
    assert "mfma_256x256" in out["eligible"] and "skinny" not in out["eligible"]


# tests/test_specializations.py:16 of the reference with the count the
# installed tree has (the one-line change INTEGRATION.md ships): five
# specializations plus hip_gemm.
COUNT_LINE = ("from specializations.catalog import list_specializations; import sys; "
              "assert len(list_specializations()) == %d; "
              "assert not any(n in sys.modules for n in ('torch', 'numpy', 'mlx'))")
REFERENCE_IDS = ("cpu_gemm", "cuda_attention", "gemmini_gemm", "metal_attention",
                 "tenstorrent_protocol")


def test_the_reference_count_assertion_reads_six_once_installed(tmp_path):
    """The installed tree holds the reference's five descriptors (its own
    files when a checkout is here, else minimal ones with the same ids) and
    hip_gemm; the catalog module is this repo's restatement of the
    reference's rules. The reference's assertion then holds with 6 and fails
    with the 5 it states today."""
    root, _ = _reference_tree(tmp_path)
    packages = root / "specializations"
    for name in REFERENCE_IDS:
        (packages / name).mkdir(exist_ok=True)
        src = os.path.join(REFERENCE, "specializations", name, "specialization.json")
        if os.path.isfile(src):
            shutil.copyfile(src, packages / name / "specialization.json")
        else:
            (packages / name / "specialization.json").write_text(
                json.dumps({"schema_version": 1, "id": name}))
    (packages / "__init__.py").write_text("")
    shutil.copyfile(os.path.join(ROOT, "veritac_amd", "specializations", "catalog.py"),
                    packages / "catalog.py")
    ids = [d["id"] for d in catalog.list_specializations(packages=str(packages))]
    assert ids == sorted(REFERENCE_IDS + ("hip_gemm",))
    proc = _run_in_tree(root, COUNT_LINE % 6, None)
    assert proc.returncode == 0, proc.stderr
    proc = _run_in_tree(root, COUNT_LINE % 5, None)
    assert proc.returncode != 0 and "AssertionError" in proc.stderr


def test_reference_side_import_fails_closed_without_the_repo(tmp_path):
    root, _ = _reference_tree(tmp_path)
    (root / "specializations" / "__init__.py").write_text("")
    proc = _run_in_tree(root, "from specializations.hip_gemm import backend", None)
    assert proc.returncode != 0 and "VT_HIP_GEMM_REPO" in proc.stderr


def test_missing_library_optimize_has_no_winner(tmp_path):
    """The reference's test_missing_checker_binary_optimize_has_no_winner
    (tests/test_gemmini.py:217-223) for the native check: with no library,
    no candidate is accepted and there is no winner."""
    code = ("import json; from veritac_amd.specializations.hip_gemm import backend as g;"
            "r = g.optimize(256, 256, 256);"
            "print(json.dumps([r['winner'], [c['check']['accepted'] for c in r['candidates']],"
            " [c['check']['reason'] for c in r['candidates'] if c['valid']]]))")
    env = dict(os.environ, VT_HIP_GEMM_LIB=str(tmp_path / "missing.so"))
    proc = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True,
                          text=True, env=env)
    assert proc.returncode == 0, proc.stderr
    winner, accepted, reasons = json.loads(proc.stdout)
    assert winner is None and accepted and not any(accepted)
    assert all("fail-closed" in r for r in reasons), reasons


@pytest.mark.parametrize("bad", ["", "HIP", "hip-gemm", "../x", None, 3, "nope"])
def test_describe_rejects_bad_ids(bad):
    with pytest.raises(ValueError):
        catalog.describe(bad)


def test_cli_list_and_show():
    out = subprocess.run([sys.executable, "-m", "veritac_amd.specializations", "show", "hip_gemm"],
                         cwd=ROOT, capture_output=True, text=True, check=True).stdout
    assert json.loads(out)["id"] == "hip_gemm"
    bad = subprocess.run([sys.executable, "-m", "veritac_amd.specializations", "show", "x/y"],
                         cwd=ROOT, capture_output=True, text=True)
    assert bad.returncode != 0

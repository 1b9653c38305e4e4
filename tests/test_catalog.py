"""The specialization catalog (mirrors the reference's tests/test_specializations.py:15-24)."""
import json
import os
import subprocess
import sys

import pytest

from veritac_amd.specializations import catalog

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


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
    d = catalog.describe("hip_gemm")
    assert d["schema_version"] == 1 and d["id"] == "hip_gemm"
    for key in ("status", "computation", "target", "implementation", "formal_sources",
                "entrypoints", "proof_scope", "boundaries", "evidence"):
        assert key in d, key
    for path in d["implementation"] + list(d["entrypoints"].values()):
        if path.endswith(".so"):
            continue   # built artefact
        assert os.path.exists(os.path.join(ROOT, path)), path


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

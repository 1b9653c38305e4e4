"""emit_c: standalone self-checking programs for hip_gemm plans (CPU side).

Mirrors the reference's EmitCTests (tests/test_gemmini.py:282-313) and its
refusal tests (:96-104, :225-240): an emitted program carries the plan, the
compile-time checks and the pass gate; invalid plans are refused before the
native check, rejected plans are refused, malformed plans raise ValueError.

Beyond that, each program is compiled here and run in --reference-only mode,
which prints a digest of the inputs it generates and of the output it expects.
The digest must equal one computed from the oracle: A and B from the oracle's
LCG (deterministic_inputs, pinned by the reference's recorded vectors), the
expected C from gemm_i8. So the program's generator and its scalar loop are
checked without a GPU. Without a device the full run must refuse (exit 2).
"""
import os
import subprocess
from unittest import mock

import numpy as np
import pytest

from oracle import gemm_oracle as go
from veritac_amd.specializations.hip_gemm import backend as hg
from veritac_amd.specializations.hip_gemm import program as pg

LIB = os.path.join(pg.LIB_DIR, "libvt_hip_gemm.so")
needs_lib = pytest.mark.skipif(not os.path.exists(LIB), reason="libvt_hip_gemm.so not built")


def fnv1a64(*chunks):
    h = 14695981039346656037
    for chunk in chunks:
        for byte in chunk:
            h ^= byte
            h = (h * 1099511628211) % 2**64
    return "%016x" % h


def oracle_digest(plan, seed, mode, *, drop_d=False):
    """Digest of (A, B, D, expected C) computed from the oracle."""
    m, n, k, batch = plan["m"], plan["n"], plan["k"], plan["batch"]
    b_mats = 1 if (plan["b_shared"] or batch == 1) else batch
    # one stream: A of every batch, then every B (the flat order of
    # deterministic_inputs with batch*m rows and b_mats*n columns)
    a, b = go.deterministic_inputs(batch * m, b_mats * n, k, seed, mode)
    A = np.array(a, np.int8).reshape(batch, m, k)
    B = np.array(b, np.int8).reshape(b_mats, k, n)   # B of batch i: rows i*k.. of the stream
    D = None
    if plan["has_d"]:
        na, nb, nc = batch * m * k, b_mats * k * n, batch * m * n
        skip = na + nb if mode == "lcg" else 0
        states = np.array(go._lcg_states(seed, skip + 2 * nc)[skip:], np.uint64)
        u = ((states[0::2] >> np.uint64(16)) << np.uint64(16)) | (states[1::2] >> np.uint64(16))
        dmax = plan["d_max_abs"]
        D = ((u % np.uint64(2 * dmax + 1)).astype(np.int64) - dmax).astype(np.int32)
        D = D.reshape(batch, m, n)
    C = np.stack([go.gemm_i8(A[i], B[i if b_mats > 1 else 0],
                             None if (D is None or drop_d) else D[i]) for i in range(batch)])
    chunks = [A.tobytes(), B.tobytes()]
    if D is not None:
        chunks.append(D.astype("<i4").tobytes())
    chunks.append(C.astype("<i4").tobytes())
    return fnv1a64(*chunks), (A, B, D)


PLANS = [
    ("config1", lambda: hg.make_plan(64, 64, 64)),
    ("config2_d", lambda: hg.make_plan(256, 256, 256, has_d=True, d_max_abs=1 << 20)),
    ("batched_shared", lambda: hg.make_plan(48, 80, 96, batch=3, b_shared=True,
                                            variant="mfma_128x128")),
    ("batched_d", lambda: hg.make_plan(16, 64, 128, batch=2, has_d=True, d_max_abs=7,
                                       variant="mfma_256x128")),
    ("skinny_split", lambda: hg.make_plan(16, 512, 1024, variant="skinny", k_split=4)),
    ("padded_shape", lambda: hg.make_plan(33, 70, 45)),
    ("packed_d", lambda: hg.make_plan(16, 256, 320, variant=hg.PACKED_VARIANT, has_d=True,
                                      d_max_abs=1000, batch=2)),
]


def build(tmp_path, plan, name, **kw):
    info = hg.emit_c(plan, str(tmp_path / (name + ".c")), **kw)
    return info, pg.build_program(info["path"])


@needs_lib
@pytest.mark.parametrize("name,make", PLANS, ids=[p[0] for p in PLANS])
def test_emission_carries_plan_checks_and_pass_gate(tmp_path, name, make):
    plan = make()
    info = hg.emit_c(plan, str(tmp_path / "p.c"))
    assert info["path"] == str(tmp_path / "p.c")
    assert info["sha256"] == hg.sha256_file(info["path"])
    assert info["counts"] == hg.modeled_counts(plan)
    text = open(info["path"]).read()
    assert "#define VERITAC_M %dLL" % plan["m"] in text
    assert "_Static_assert(VT_ABI_VERSION == 7" in text
    assert "k*16384 + d_max_abs > 2^31-1" in text
    assert pg.PASS_MARKER in text and pg.FAIL_MARKER in text
    assert ("vt_gemm_i8_packed(" if plan["variant"] == hg.PACKED_VARIANT else "vt_gemm_i8(") in text
    assert "ANALYTIC MODELS, not measurements" in text


@needs_lib
@pytest.mark.parametrize("name,make", PLANS, ids=[p[0] for p in PLANS])
def test_program_inputs_and_expected_output_match_the_oracle(tmp_path, name, make):
    plan = make()
    seed = 0x12345678 if name != "batched_d" else 7
    _, exe = build(tmp_path, plan, name, seed=seed)
    out = subprocess.run([exe, "--reference-only"], capture_output=True, text=True, check=True)
    got = out.stdout.split()[-1]
    want, (A, B, D) = oracle_digest(plan, seed, "lcg")
    assert got == want
    # the package's mirror of the generator agrees with the oracle's stream
    pa, pb, pd = pg.program_inputs(plan, seed)
    assert np.array_equal(pa, A) and np.array_equal(pb, B)
    assert (pd is None and D is None) or np.array_equal(pd, D)
    if D is not None:
        assert np.abs(D).max() <= plan["d_max_abs"]
        # planted mistake in the oracle: D left out of the expected output
        assert oracle_digest(plan, seed, "lcg", drop_d=True)[0] != got
    # planted mistake: the stream started one step late
    assert oracle_digest(plan, seed + 1, "lcg")[0] != got


@needs_lib
@pytest.mark.parametrize("mode", ["max", "minmax", "min", "zero"])
@pytest.mark.parametrize("has_d", [True, False])
def test_constant_modes_match_the_oracle(tmp_path, mode, has_d):
    plan = hg.make_plan(32, 48, 8192, has_d=has_d, d_max_abs=5 if has_d else 0,
                        variant="generic")
    _, exe = build(tmp_path, plan, mode, input_mode=mode)
    out = subprocess.run([exe, "--reference-only"], capture_output=True, text=True, check=True)
    assert out.stdout.split()[-1] == oracle_digest(plan, pg.DEFAULT_SEED, mode)[0]


@needs_lib
def test_full_run_without_a_device_refuses(tmp_path):
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible: the device run is covered by the -m gpu tests")
    _, exe = build(tmp_path, hg.make_plan(64, 64, 64), "nodev")
    out = subprocess.run([exe], capture_output=True, text=True)
    assert out.returncode == 2
    assert "no gfx950 device visible" in out.stdout
    assert pg.FAIL_MARKER in out.stdout and pg.PASS_MARKER not in out.stdout


def test_invalid_plan_is_refused_before_the_native_check(tmp_path):
    plan = hg.make_plan(32, 32, 32, variant="mfma_128x128")
    plan["k"] = 33   # not divisible by 16
    with mock.patch.object(pg, "native_check") as never:
        with pytest.raises(ValueError):
            hg.emit_c(plan, str(tmp_path / "bad.c"))
        never.assert_not_called()
    assert not (tmp_path / "bad.c").exists()


def test_malformed_plan_object_is_refused(tmp_path):
    with pytest.raises(ValueError):
        hg.emit_c(["not", "a", "dict"], str(tmp_path / "notdict.c"))


def test_native_rejection_blocks_emission(tmp_path):
    plan = hg.make_plan(64, 64, 64)
    with mock.patch.object(pg, "native_check", return_value=(False, "mocked rejection")):
        with pytest.raises(ValueError, match="mocked rejection"):
            hg.emit_c(plan, str(tmp_path / "rejected.c"))
    assert not (tmp_path / "rejected.c").exists()


@pytest.mark.parametrize("kw", [dict(input_mode="random"), dict(seed=-1), dict(seed=2**32),
                                dict(seed=1.5)])
def test_bad_seed_or_mode_is_refused(tmp_path, kw):
    with pytest.raises(ValueError):
        hg.emit_c(hg.make_plan(64, 64, 64), str(tmp_path / "x.c"), **kw)


def test_reference_side_backend_exports_emit_c(monkeypatch):
    monkeypatch.setenv("VT_HIP_GEMM_REPO", os.path.dirname(pg.LIB_DIR))
    from veritac_amd.specializations.hip_gemm.reference_side import backend as ref_side
    assert ref_side.emit_c is hg.emit_c and ref_side.sha256_file is hg.sha256_file

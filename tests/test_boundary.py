"""C-ABI boundary on a host without a GPU: the library loads, exports every
symbol include/vt_hip_gemm.h declares, validates arguments before any device
call, and fails closed (VT_ENODEV) when no gfx950 device exists."""
import ctypes
import os
import re

import pytest

import veritac_amd
from veritac_amd import _lib
from veritac_amd.specializations.hip_gemm import backend as hg

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vt_hip_gemm.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vt_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = veritac_amd.load_library()
    declared = header_functions()
    assert declared == sorted(_lib.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name
    header = open(os.path.join(ROOT, "include", "vt_hip_gemm.h")).read()
    assert "#define VT_ABI_VERSION %d" % _lib.ABI_VERSION in header
    assert lib.vt_abi_version() == _lib.ABI_VERSION


def test_variant_table_matches_backend():
    for name in hg.VARIANTS:
        info = _lib.variant_info(name)
        assert (info["tile_m"], info["tile_n"], info["tile_k"], info["threads"],
                info["lds_bytes"]) == hg.TILES[name], name
        assert veritac_amd.load_library().vt_variant_name(_lib.VARIANT_IDS[name]).decode() == name
    assert veritac_amd.load_library().vt_variant_name(99) is None


def test_native_selection_for_benchmark_configs():
    assert _lib.select_variant(16, 14336, 4096)[0] == "skinny"
    assert _lib.select_variant(1, 14336, 4096)[0] == "skinny"
    assert _lib.select_variant(8192, 8192, 8192) == ("mfma_256x256", 0)
    assert _lib.select_variant(512, 1024, 1024, 64)[0].startswith("mfma")
    # tiny problems (M > 16, K <= 64, at most 2^20 multiply-adds) run on the VALU kernel
    assert _lib.select_variant(64, 64, 64)[0] == "generic"
    assert _lib.select_variant(64, 256, 64)[0] == "generic"                      # exactly 2^20
    assert _lib.select_variant(64, 272, 64)[0] == "mfma_128x128"
    assert _lib.select_variant(16, 256, 64)[0] == "skinny"
    assert _lib.select_variant(128, 128, 128)[0] == "mfma_128x128"
    # 17..64 rows with K >= 512: one B stream on the skinny kernel's row blocks,
    # unless 128-column tiles alone fill the chip
    assert _lib.select_variant(64, 14336, 4096)[0] == "skinny"
    assert _lib.select_variant(17, 4096, 4096)[0] == "skinny"
    assert _lib.select_variant(64, 28672, 8192)[0] == "skinny"
    assert _lib.select_variant(64, 32768, 1024)[0] == "mfma_128x128"     # 256 tiles
    assert _lib.select_variant(64, 4096, 256)[0] == "mfma_128x128"       # short K
    assert _lib.select_variant(65, 4096, 4096)[0] == "mfma_128x128"
    assert _lib.select_variant(64, 60, 64, aligned=False)[0] == "generic"


def call(M=4, N=16, K=16, lda=None, ldb=None, ldd=None, ldc=None, batch=1, variant=0,
         k_split=0, A=1 << 20, B=1 << 21, D=None, C=1 << 22, strides=(0, 0, 0, 0)):
    lib = veritac_amd.load_library()
    return lib.vt_gemm_i8(A, B, D, C, M, N, K, K if lda is None else lda,
                          N if ldb is None else ldb, N if ldd is None else ldd,
                          N if ldc is None else ldc, batch, *strides, variant, k_split, None)


@pytest.mark.parametrize("kw", [
    dict(M=-1), dict(N=-2), dict(K=-3), dict(batch=-1), dict(C=None), dict(A=None),
    dict(B=None), dict(lda=8), dict(ldb=8), dict(ldc=8), dict(D=1 << 23, ldd=4),
    dict(variant=99), dict(k_split=-1), dict(batch=2, strides=(64, 0, 0, 0)),
    dict(strides=(-16, 0, 0, 0)),
])
def test_invalid_arguments_rejected_before_device(kw):
    assert call(**kw) == _lib.VT_EINVAL
    assert _lib.last_error()


def test_explicit_vector_variant_refuses_unaligned_shapes():
    assert call(N=20, variant=1) == _lib.VT_EUNSUPPORTED
    assert call(K=20, lda=20, variant=3) == _lib.VT_EUNSUPPORTED
    assert call(M=65, variant=3) == _lib.VT_EUNSUPPORTED
    assert call(A=(1 << 20) + 1, variant=2) == _lib.VT_EUNSUPPORTED


def test_empty_problems_are_noops():
    assert call(M=0, C=None, A=None, B=None) == _lib.VT_OK
    assert call(N=0, C=None) == _lib.VT_OK
    assert call(batch=0) == _lib.VT_OK


@pytest.mark.skipif(veritac_amd.load_library().vt_device_count() > 0, reason="GPU present")
def test_fails_closed_without_gpu():
    assert veritac_amd.load_library().vt_device_count() == 0
    assert call() == _lib.VT_ENODEV
    assert "device" in _lib.last_error()
    assert veritac_amd.load_library().vt_sync(None) == _lib.VT_ENODEV
    with pytest.raises(_lib.HipGemmError):
        _lib.gemm_raw(1 << 20, 1 << 21, None, 1 << 22, 4, 16, 16, 16, 16, 16, 16)


def test_missing_library_fails_closed(tmp_path, monkeypatch):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setenv("VT_HIP_GEMM_LIB", str(tmp_path / "nope.so"))
    with pytest.raises(_lib.HipGemmError):
        _lib.load_library()
    bad = tmp_path / "bad.so"
    bad.write_bytes(b"not an ELF")
    monkeypatch.setenv("VT_HIP_GEMM_LIB", str(bad))
    with pytest.raises(_lib.HipGemmError):
        _lib.load_library()
    monkeypatch.delenv("VT_HIP_GEMM_LIB")
    monkeypatch.setattr(_lib, "_lib", None)
    assert _lib.load_library() is not None


REPLAY_OK = dict(prog=1 << 20, n_ops=1, A=1 << 21, B=1 << 22, C=1 << 23, m=16, n=16, k=16,
                 sp=32, acc=16, status=1 << 24)


@pytest.mark.parametrize("kw", [dict(m=0), dict(k=-16), dict(n_ops=-1), dict(sp=8), dict(acc=15),
                                dict(A=None), dict(status=None), dict(prog=None),
                                dict(m=1 << 20, k=1 << 20)])
def test_replay_invalid_arguments_rejected_before_device(kw):
    a = dict(REPLAY_OK, **kw)
    lib = veritac_amd.load_library()
    rc = lib.vt_replay_i8(a["prog"], a["n_ops"], a["A"], a["B"], a["C"], a["m"], a["n"], a["k"],
                          a["sp"], a["acc"], a["status"], None)
    assert rc == _lib.VT_EINVAL, _lib.last_error()


def test_replay_refuses_a_scratchpad_beyond_lds():
    a = dict(REPLAY_OK, sp=16384, acc=1024)
    lib = veritac_amd.load_library()
    rc = lib.vt_replay_i8(a["prog"], a["n_ops"], a["A"], a["B"], a["C"], a["m"], a["n"], a["k"],
                          a["sp"], a["acc"], a["status"], None)
    assert rc == _lib.VT_EUNSUPPORTED and "LDS" in _lib.last_error()


def test_replay_fails_closed_without_gpu():
    if _lib.device_count() > 0:
        pytest.skip("a gfx950 device is present")
    a = REPLAY_OK
    with pytest.raises(_lib.HipGemmError) as exc:
        _lib.replay_raw(a["prog"], a["n_ops"], a["A"], a["B"], a["C"], a["m"], a["n"], a["k"],
                        a["sp"], a["acc"], a["status"])
    assert exc.value.code == _lib.VT_ENODEV


def test_device_info_layout_matches_the_header(tmp_path):
    """The ctypes structure has the C compiler's size and field offsets."""
    fields = [name for name, _ in _lib.DeviceInfo._fields_]
    src = tmp_path / "layout.c"
    src.write_text("#include <stddef.h>\n#include <stdio.h>\n#include \"vt_hip_gemm.h\"\n"
                   "int main(void) {\n  printf(\"%zu\\n\", sizeof(vt_device_info));\n" +
                   "".join('  printf("%%zu\\n", offsetof(vt_device_info, %s));\n' % f
                           for f in fields) + "  return 0;\n}\n")
    exe = tmp_path / "layout"
    import subprocess
    subprocess.run(["gcc", "-std=c99", "-I", os.path.join(ROOT, "include"), str(src), "-o",
                    str(exe)], check=True)
    out = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True,
                                          check=True).stdout.split()]
    assert out[0] == ctypes.sizeof(_lib.DeviceInfo)
    assert out[1:] == [getattr(_lib.DeviceInfo, f).offset for f in fields]
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    body = re.search(r"typedef struct vt_device_info \{(.*?)\}", text, flags=re.S).group(1)
    assert re.findall(r"(\w+)(?:\[\d+\])?;", body) == fields


def test_device_query_validates_before_the_runtime():
    lib = veritac_amd.load_library()
    info = _lib.DeviceInfo()
    assert lib.vt_device_query(-1, None, ctypes.sizeof(info)) == _lib.VT_EINVAL
    assert lib.vt_device_query(-1, ctypes.byref(info), ctypes.sizeof(info) - 8) == _lib.VT_EINVAL
    assert "info_size" in _lib.last_error()


def test_device_query_fails_closed_without_gpu():
    if _lib.device_count() > 0:
        pytest.skip("a gfx950 device is present")
    with pytest.raises(_lib.HipGemmError) as exc:
        _lib.device_query()
    assert exc.value.code == _lib.VT_ENODEV


# ---------------------------------------------------------------------------
# Extents and overlapping operands (refused on the host, before any device call)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("kw", [
    dict(lda=1 << 41), dict(ldc=1 << 41), dict(batch=2, strides=(0, 0, 0, 1 << 57)),
    dict(M=1 << 41), dict(batch=1 << 32, strides=(0, 0, 0, 64)),
    # M * ldc would overflow 64 bits in the stride check
    dict(M=1 << 30, ldc=1 << 40, batch=2, strides=(0, 0, 0, 1 << 50)),
])
def test_extents_beyond_the_address_space_are_refused(kw):
    assert call(**kw) == _lib.VT_EINVAL
    assert _lib.last_error()


def test_output_may_not_overlap_an_input():
    # A at 1<<20 spans 4*16 bytes; C at 1<<20 + 32 overlaps it
    assert call(C=(1 << 20) + 32) == _lib.VT_EINVAL
    assert "overlaps A or B" in _lib.last_error()
    assert call(C=(1 << 21) + 64) == _lib.VT_EINVAL          # inside B (16 x 16 bytes)
    # D partially overlapping C
    assert call(D=(1 << 22) + 64) == _lib.VT_EINVAL
    assert "D overlaps C" in _lib.last_error()
    # D == C but another leading dimension: not in place, refused
    assert call(D=1 << 22, ldd=32, ldc=16) == _lib.VT_EINVAL
    # batched: D == C with a different batch stride
    assert call(D=1 << 22, batch=2, strides=(64, 0, 128, 64 * 4)) == _lib.VT_EINVAL


@pytest.mark.skipif(veritac_amd.load_library().vt_device_count() > 0, reason="GPU present")
def test_in_place_and_adjacent_operands_pass_validation():
    # exact in place (same base, ld and stride) and operands that merely touch
    # pass the host checks and reach the device query (no device here)
    assert call(D=1 << 22) == _lib.VT_ENODEV
    assert call(D=1 << 22, batch=2, strides=(64, 0, 256, 256)) == _lib.VT_ENODEV
    assert call(C=(1 << 20) + 64) == _lib.VT_ENODEV            # right after A (4 x 16 bytes)


def test_packed_entry_points_refuse_overlap():
    lib = veritac_amd.load_library()
    size = _lib.packed_b_size(64, 16)
    # pack: Bp inside B
    rc = lib.vt_pack_b_i8(1 << 20, (1 << 20) + 512, 64, 16, 16, 1, 0, 0, None)
    assert rc == _lib.VT_EINVAL and "overlaps" in _lib.last_error()
    # packed GEMM: C over the packed B
    rc = lib.vt_gemm_i8_packed(1 << 20, 1 << 21, None, (1 << 21) + 16, 4, 16, 64, 64, 16, 16,
                               1, 0, 0, 0, 0, 0, None)
    assert rc == _lib.VT_EINVAL and "overlaps" in _lib.last_error()
    assert size == 1024


def test_padded_variant_selection_and_refusals():
    # unaligned shapes: the padded path from 3 * 2^24 multiply-adds, the VALU kernel below
    assert _lib.select_variant(1000, 1000, 1000, aligned=False) == ("padded", 0)
    assert _lib.select_variant(48, 1024, 1024, aligned=False)[0] == "padded"      # exactly 3 * 2^24
    assert _lib.select_variant(47, 1024, 1024, aligned=False)[0] == "generic"
    assert _lib.select_variant(17, 14335, 4095, aligned=False)[0] == "padded"
    assert _lib.select_variant(1 << 30, 16, 16, aligned=False)[0] == "generic"     # M too large
    # an explicit padded call is validated like any other before the device
    assert call(variant=6, M=-1) == _lib.VT_EINVAL
    assert call(variant=6, C=(1 << 20) + 8) == _lib.VT_EINVAL                    # C over A


# ---------------------------------------------------------------------------
# vt_gemm_check: the native acceptance check, no device needed
# ---------------------------------------------------------------------------

def test_gemm_check_accepts_and_resolves_the_benchmark_configs():
    assert _lib.gemm_check(8192, 8192, 8192, 8192, 8192, 8192, 8192) == (
        0, "ok", "mfma_256x256", 0, 0)
    st, _, v, ks, ws = _lib.gemm_check(16, 14336, 4096, 4096, 14336, 14336, 14336)
    assert (st, v, ks) == (0, "skinny", 4) and ws == 4 * 16 * 14336 * 4
    # config 3: shared B folds into one GEMM with stacked M
    st, _, v, _, ws = _lib.gemm_check(512, 1024, 1024, 1024, 1024, 1024, 1024, batch=64,
                                      stride_a=512 * 1024, stride_b=0, stride_c=512 * 1024)
    assert (st, v, ws) == (0, "mfma_256x256", 0)
    # nothing to compute
    assert _lib.gemm_check(0, 16, 16, 16, 16, 16, 16)[:3] == (0, "ok", "auto")


def test_gemm_check_refusals_carry_the_native_reason():
    st, reason, *_ = _lib.gemm_check(16, 14336, 4095, 4095, 14336, 14336, 14336, variant="skinny")
    assert st == _lib.VT_EUNSUPPORTED and "K%16==0" in reason
    st, reason, *_ = _lib.gemm_check(32, 16, 16, 8, 16, 16, 16)
    assert st == _lib.VT_EINVAL and "lda" in reason
    st, reason, *_ = _lib.gemm_check(32, 16, 16, 16, 16, 16, 16, batch=2, stride_c=16)
    assert st == _lib.VT_EINVAL and "stride_c" in reason
    st, reason, *_ = _lib.gemm_check(32, 16, 16, 16, 16, 8, 16, has_d=True)
    assert st == _lib.VT_EINVAL and "ldd" in reason
    st, reason, *_ = _lib.gemm_check(65, 16, 16, 16, 16, 16, 16, variant="skinny")
    assert st == _lib.VT_EUNSUPPORTED and "M <= 64" in reason


def test_mfma_variant_refuses_rows_too_long_for_tile_offsets():
    """256 * lda >= 2^32: an explicit MFMA variant refuses (no silent VALU
    run); auto picks the VALU kernel past the skinny kernel's 64 rows (that
    kernel addresses A and B with 64-bit offsets), and the check says which."""
    k = 1 << 24
    for variant in ("mfma_256x256", "mfma_256x128", "mfma_128x128"):
        st, reason, *_ = _lib.gemm_check(100, 64, k, k, 64, 64, 64, variant=variant)
        assert st == _lib.VT_EUNSUPPORTED and "256*lda" in reason, variant
    st, _, chosen, _, _ = _lib.gemm_check(100, 64, k, k, 64, 64, 64)
    assert st == 0 and chosen == "generic"
    assert _lib.select_variant(100, 64, k)[0] == "generic"
    assert _lib.select_variant(32, 64, k)[0] == "skinny"
    # below the limit the MFMA variants accept rows of any length
    k = (1 << 24) - 4096
    assert _lib.gemm_check(32, 64, k, k, 64, 64, 64, variant="mfma_128x128")[0] == 0


def test_gemm_check_reports_padded_and_skinny_workspace():
    # padded: A and B copied with K and N rounded to 16, C copied out
    st, _, v, _, ws = _lib.gemm_check(1000, 1000, 1000, 1000, 1000, 1000, 1000)
    assert (st, v) == (0, "padded")
    r256 = lambda x: -(-x // 256) * 256
    assert ws == r256(1000 * 1008) + r256(1008 * 1008) + r256(1000 * 1008 * 4)
    # explicit k_split of the skinny kernel
    st, _, v, ks, ws = _lib.gemm_check(16, 2048, 4096, 4096, 2048, 2048, 2048, variant="skinny",
                                       k_split=8)
    assert (st, v, ks) == (0, "skinny", 8) and ws == 8 * 16 * 2048 * 4


def test_select_follows_b_sharing():
    """The fold into a stacked-M GEMM needs one shared B: with per-batch B
    the selection is the one vt_gemm_i8 makes for unshared batches (two
    batches of 64 rows: 400 tiles of 256x256, against 128 stacked rows on
    128x128 tiles)."""
    shared = _lib.select_variant(64, 51200, 128, 2, b_shared=True)
    unshared = _lib.select_variant(64, 51200, 128, 2, b_shared=False)
    assert shared == ("mfma_128x128", 0) and unshared == ("mfma_256x256", 0)
    assert _lib.gemm_check(64, 51200, 128, 128, 51200, 51200, 51200, batch=2,
                           stride_a=64 * 128, stride_b=128 * 51200,
                           stride_c=64 * 51200)[2] == unshared[0]
    assert _lib.gemm_check(64, 51200, 128, 128, 51200, 51200, 51200, batch=2,
                           stride_a=64 * 128, stride_b=0,
                           stride_c=64 * 51200)[2] == shared[0]
    assert hg.make_plan(64, 51200, 128, batch=2)["variant"] == unshared[0]
    assert hg.make_plan(64, 51200, 128, batch=2, b_shared=True)["variant"] == shared[0]
    lib = veritac_amd.load_library()
    v, ks = ctypes.c_int32(), ctypes.c_int32()
    assert lib.vt_gemm_select(16, 16, 16, 1, 16, 16, 4, ctypes.byref(v), ctypes.byref(ks)) \
        == _lib.VT_EINVAL


def test_optimize_candidates_carry_the_native_check():
    """Each candidate has the reference's keys (backend.py:1083-1085); only
    valid, accepted candidates are scored; the winner is one of them."""
    r = hg.optimize(16, 14336, 4096)
    keys = {"plan", "valid", "invalid_reason", "check", "counts", "objective"}
    for c in r["candidates"]:
        assert keys <= set(c)
        assert set(c["check"]) == {"accepted", "reason"}
        if c["valid"] and c["check"]["accepted"]:
            assert c["objective"] is not None and "vt_gemm_check" in c["check"]["reason"]
        else:
            assert c["objective"] is None
    assert r["winner"]["variant"] == "skinny"
    # a plan the Python validation accepts but the native check refuses
    plan = dict(hg.make_plan(16, 64, 64), variant="mfma_128x128", k=1 << 24)
    assert hg.native_check(plan)[0] is False

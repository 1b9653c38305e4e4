"""hip_gemm backend host logic on the CPU: plan validation (mirrors the
reference's tests/test_gemmini.py:96-161 and test_gemmini_checker.py:26-67),
candidate selection, input generators, and fail-closed execution with an
injected runner."""
import numpy as np
import pytest
import torch

from oracle import gemm_oracle as go
from veritac_amd import HipGemmError
from veritac_amd.specializations.hip_gemm import backend as hg
from veritac_amd.specializations.hip_gemm import inputs


def plan(**kw):
    p = hg.make_plan(32, 32, 32, variant="mfma_128x128")
    p.update(kw)
    return p


def test_minimum_plans_validate():
    for v in hg.VARIANTS:
        for shape in ((16, 16, 16), (32, 32, 32), (48, 32, 64)):
            if v == "skinny":
                shape = (min(shape[0], 16),) + shape[1:]
            p = hg.make_plan(*shape, variant=v)
            ok, reason = hg.validate_plan(p)
            assert ok, (v, shape, reason)


@pytest.mark.parametrize("name", ["m", "n", "k", "batch", "dim", "d_max_abs", "k_split"])
@pytest.mark.parametrize("value", [0.5, True, None, "32", [], {}])
def test_malformed_integer_fields_rejected(name, value):
    ok, reason = hg.validate_plan(plan(**{name: value}))
    assert not ok and name in reason


def test_missing_fields_and_non_dict_rejected():
    for name in ("m", "n", "k", "batch", "dim", "variant", "has_d", "b_shared"):
        p = plan()
        del p[name]
        assert not hg.validate_plan(p)[0]
    for value in (None, [], "plan", 42):
        assert hg.validate_plan(value) == (False, "plan must be a JSON object")
    assert not hg.validate_plan(plan(has_d=1))[0]


@pytest.mark.parametrize("changes", [dict(m=0), dict(n=0), dict(k=0), dict(dim=0), dict(dim=8),
                                     dict(n=17), dict(k=33), dict(k=131072), dict(batch=0),
                                     dict(variant="unknown"), dict(variant="auto"),
                                     dict(k_split=-1), dict(k_split=2), dict(d_max_abs=5)])
def test_bad_shapes_and_arithmetic_bound(changes):
    assert not hg.validate_plan(plan(**changes))[0]


def test_overflow_bound_boundary():
    # k*16384 <= 2^31-1 (Plan.lean:86-92): k=131056 accepted, k=131072 rejected
    assert hg.validate_plan(plan(k=131056))[0]
    assert not hg.validate_plan(plan(k=131072))[0]
    # with an initial partial sum the bound includes |D|
    assert hg.validate_plan(plan(k=256, has_d=True, d_max_abs=1 << 20))[0]
    assert not hg.validate_plan(plan(k=131056, has_d=True, d_max_abs=1 << 20))[0]


def test_variant_specific_rules():
    assert hg.validate_plan(plan(m=1, variant="skinny"))[0]
    assert hg.validate_plan(plan(m=16, variant="skinny", k_split=3))[0]
    assert hg.validate_plan(plan(m=64, variant="skinny"))[0]     # 4 row blocks of 16
    assert not hg.validate_plan(plan(m=65, variant="skinny"))[0]
    assert hg.validate_plan(plan(m=5, n=7, k=9, variant="generic"))[0]
    assert not hg.validate_plan(plan(m=5, n=7, k=9, variant="mfma_256x256"))[0]


def test_make_plan_auto_and_optimize():
    p = hg.make_plan(16, 14336, 4096)
    assert p["variant"] == "skinny" and p["k_split"] >= 1
    assert hg.make_plan(8192, 8192, 8192)["variant"] == "mfma_256x256"
    assert hg.make_plan(5, 7, 9)["variant"] == "generic"
    res = hg.optimize(8192, 8192, 8192)
    names = [c["plan"]["variant"] for c in res["candidates"]]
    assert names == list(hg.VARIANTS)
    skinny = res["candidates"][names.index("skinny")]
    assert not skinny["valid"] and "m <= 64" in skinny["invalid_reason"]
    assert res["winner"]["variant"] == "mfma_256x256"
    res = hg.optimize(16, 14336, 4096)
    assert res["winner"]["variant"] == "skinny"
    with pytest.raises(HipGemmError):
        hg.make_plan(0, 16, 16)


def test_modeled_counts_are_consistent():
    p = hg.make_plan(64, 512, 1024, batch=64, b_shared=True, variant="mfma_256x256")
    c = hg.modeled_counts(p)
    assert c["ops"] == 2 * 64 * 64 * 512 * 1024
    assert c["bytes_algorithmic"] == 64 * 64 * 1024 + 1024 * 512 + 4 * 64 * 64 * 512
    # 32 tiles of a K of 1024: two K slices of 512
    assert hg.mfma_k_split(p) == 2
    assert c["workgroups"] == (64 * 64 // 256) * (512 // 256) * 2
    p = hg.make_plan(256, 256, 256, has_d=True, d_max_abs=1 << 20, variant="mfma_128x128")
    assert hg.modeled_counts(p)["bytes_algorithmic"] == 2 * 65536 + 8 * 65536


def test_skinny_split_mirrors_native_rule():
    p = hg.make_plan(16, 14336, 4096, variant="skinny")
    ks, chunk = hg.skinny_split(p)
    assert (ks, chunk) == (4, 1024)          # 56 column slabs x 4 K slices
    for req in (1, 2, 3, 4, 7):
        ks, chunk = hg.skinny_split(dict(p, k_split=req))
        assert chunk % hg.SKINNY_PIPE_ROWS == 0 and ks * chunk >= 4096 and (ks - 1) * chunk < 4096
    p = hg.make_plan(16, 2048, 8192, variant="skinny")    # 8 slabs: split K
    ks, chunk = hg.skinny_split(p)
    assert ks == 22 and chunk == 384        # 28 requested -> 384-row slices
    p = hg.make_plan(16, 65536, 4096, variant="skinny")   # 256 slabs: no split
    assert hg.skinny_split(p) == (1, 4096)
    lds, wgs = hg.required_resources(dict(p, k=131056, k_split=1))
    assert lds <= hg.LDS_PER_CU


def fake_runner(plan, A, B, D, C, stream):
    """Host-side stand-in for the device: computes through the oracle (tests only)."""
    out = go.gemm_i8(A.numpy(), B.numpy(), None if D is None else D.numpy())
    C.copy_(torch.from_numpy(out))


def test_run_with_injected_runner():
    A, B = inputs.deterministic_inputs(32, 48, 64, 7)
    p = hg.make_plan(32, 48, 64, variant="mfma_128x128")
    C = hg.run(p, torch.from_numpy(A), torch.from_numpy(B), runner=fake_runner)
    assert np.array_equal(C.numpy(), go.gemm_i8(A, B))


def test_run_fails_closed():
    A = torch.zeros(32, 32, dtype=torch.int8)
    B = torch.zeros(32, 32, dtype=torch.int8)
    p = plan()
    with pytest.raises(HipGemmError, match="no CPU path"):
        hg.run(p, A, B)                                  # CPU tensors, no runner
    with pytest.raises(HipGemmError, match="invalid plan"):
        hg.run(plan(k=33), A, B, runner=fake_runner)
    with pytest.raises(HipGemmError, match="shape"):
        hg.run(plan(n=48), A, B, runner=fake_runner)
    with pytest.raises(HipGemmError, match="int8"):
        hg.run(p, A.int(), B, runner=fake_runner)
    with pytest.raises(HipGemmError, match="D"):
        hg.run(p, A, B, D=torch.zeros(32, 32, dtype=torch.int32), runner=fake_runner)
    with pytest.raises(HipGemmError, match="has_d"):
        hg.run(plan(has_d=True, d_max_abs=1), A, B, runner=fake_runner)
    with pytest.raises(HipGemmError, match="unit stride"):
        hg.run(p, A.t(), B, runner=fake_runner)


def test_run_flat_validates_like_the_interpreter():
    p = hg.make_plan(16, 16, 16, variant="generic")
    with pytest.raises(HipGemmError, match="out of"):
        hg.run_flat(p, [200] * 256, [0] * 256)
    with pytest.raises(HipGemmError, match="values"):
        hg.run_flat(p, [0] * 10, [0] * 256)
    with pytest.raises(HipGemmError):
        hg.run_flat(p, [1.0] * 256, [0] * 256)


def test_product_generators_match_oracle():
    for mode in ("lcg", "max", "minmax", "min", "zero"):
        for seed in (0, 7, 917, 987654321):
            A, B = inputs.deterministic_inputs(5, 9, 6000 if mode == "lcg" and seed == 7 else 3,
                                               seed, mode)
            oa, ob = go.deterministic_inputs(A.shape[0], B.shape[1], A.shape[1], seed, mode)
            assert A.reshape(-1).tolist() == oa and B.reshape(-1).tolist() == ob
    for mode in ("zeros", "extrema", "lcg"):
        A, B = inputs.spike_inputs(mode, 16, 32, 48)
        a, b = go.fill_inputs(mode, 16 * 48, 48 * 32)
        assert A.reshape(-1).tolist() == [go.to_int8(v) for v in a]
        assert B.reshape(-1).tolist() == [go.to_int8(v) for v in b]


def test_config_inputs_properties():
    c1 = inputs.config_inputs(1, seed=1)
    assert c1["A"].shape == (64, 64) and c1["D"] is None and c1["A"].dtype == np.int8
    c2 = inputs.config_inputs(2, seed=1)
    assert c2["D"].dtype == np.int32 and np.abs(c2["D"].astype(np.int64)).max() <= 1 << 20
    c3 = inputs.config_inputs(3, seed=1)
    assert c3["A"].shape == (64, 512, 1024) and c3["B"].shape == (1024, 1024)
    c4 = inputs.config_inputs(4, seed=1, m=1)
    assert c4["A"].shape == (1, 4096) and c4["A"].min() >= -127
    assert c4["B"].shape == (4096, 14336) and 25 < c4["B"].astype(np.float64).std() < 39
    again = inputs.config_inputs(2, seed=1)
    assert np.array_equal(again["A"], c2["A"]) and np.array_equal(again["D"], c2["D"])
    assert inputs.config_shape(5) == (1, 8192, 8192, 8192, False, False)


def test_padded_plans_take_any_n_and_k():
    p = hg.make_plan(1000, 1000, 1000)
    assert p["variant"] == "padded" and hg.validate_plan(p) == (True, "ok")
    inner = hg.padded_inner_plan(p)
    assert (inner["n"], inner["k"]) == (1008, 1008) and inner["variant"].startswith("mfma")
    assert not inner["has_d"]
    p = hg.make_plan(16, 14335, 4095, variant="padded")
    assert hg.validate_plan(p)[0] and hg.padded_inner_plan(p)["variant"] == "skinny"
    assert hg.validate_plan(dict(p, k_split=2)) == (False, "variant 'padded' chooses its own k_split (give 0)")
    assert not hg.validate_plan(dict(p, batch=70000))[0]
    # only operands the vector kernels cannot read as they are get copied, and
    # with n % 16 == 0 the product writes C and adds D itself (no copy-out)
    p = hg.make_plan(3000, 2000, 1500, has_d=True, d_max_abs=5, variant="padded")
    assert hg._padded_copies(p) == (True, True, False)
    inner = hg.padded_inner_plan(p)
    assert inner["has_d"] and inner["d_max_abs"] == 5 and (inner["n"], inner["k"]) == (2000, 1504)
    assert hg._padded_copy_bytes(p, inner) < 3000 * 2000 * 4              # no C traffic priced
    assert hg._padded_copies(hg.make_plan(300, 1001, 1024, variant="padded")) == (False, True, True)
    assert hg._padded_copies(hg.make_plan(256, 256, 256, variant="padded")) == (False, False, False)
    # small unaligned shapes stay on the VALU kernel; aligned shapes never pick padded
    assert hg.make_plan(64, 60, 64)["variant"] == "generic"
    assert hg.optimize(1024, 1024, 1024)["winner"]["variant"].startswith("mfma")
    counts = hg.modeled_counts(hg.make_plan(1000, 1000, 1000, has_d=True, d_max_abs=7))
    assert counts["bytes_l2_modeled"] > counts["bytes_algorithmic"]


def test_mfma_k_split_mirrors_the_native_choice():
    """Few long MFMA tiles run as K slices plus a reduction; the plan mirror
    reports the same split as vt_gemm_check and sizes workgroups with it."""
    from veritac_amd import _lib
    for m, n, k in [(128, 14336, 4096), (96, 14336, 4096), (128, 4096, 4096), (256, 4096, 4096),
                    (512, 4096, 4096), (8192, 8192, 8192), (1024, 14336, 4096), (300, 208, 160),
                    (128, 4096, 1024), (128, 4096, 1152), (100, 256, 65536), (96, 2048, 1024),
                    (256, 256, 8192), (768, 2048, 8192), (512, 4096, 16384), (768, 2048, 4096),
                    (1280, 2048, 8192)]:
        plan = hg.make_plan(m, n, k)
        _, _, variant, ks, ws = _lib.gemm_check(m, n, k, k, n, n, n)
        assert plan["variant"] == variant
        want = ks if ks > 1 else 1
        assert hg.mfma_k_split(plan) == want, (m, n, k)
        if variant.startswith("mfma"):
            # small mfma_128x128 grids run 64x128 or 64x64 tiles (pinned by
            # test_small_128x128_grids_run_smaller_tiles)
            tm, tn = hg.mfma_tile_shape(plan)
            tiles = -(-m // tm) * -(-n // tn) * want
            assert hg.mfma_tiles(plan) == tiles
            persistent = (variant == "mfma_256x256" and m >= 256 and n >= 256 and
                          (k // want) % 64 == 0) or \
                (variant == "mfma_256x128" and m >= 256 and n >= 128 and
                 (k // want) % 256 == 0)
            # the persistent kernel: one workgroup per CU, 160 KiB (K slice % 256
            # == 0) or 128 KiB of LDS; the tile kernel: a workgroup per tile
            lds = 3 * (tm * 64 + 64 * tn) if tm == 64 else hg.TILES[variant][4]
            assert hg.required_resources(plan) == (
                (hg.DMA16_LDS if (k // want) % 256 == 0 else hg.DMA_LDS, min(tiles, 256))
                if persistent else (lds, tiles)), (m, n, k)
            assert ws == (want * m * n * 4 if want > 1 else 0)
    assert hg.mfma_k_split(hg.make_plan(128, 4096, 4096)) == 4     # on 64x128 tiles
    assert hg.mfma_k_split(hg.make_plan(128, 4096, 8192)) == 8     # on 128x128 tiles
    assert hg.mfma_k_split(hg.make_plan(128, 4096, 1024)) == 1     # 128 64x64 workgroups
    assert hg.mfma_k_split(hg.make_plan(96, 2048, 1024)) == 2      # slices of 512
    assert hg.mfma_k_split(hg.make_plan(128, 4096, 1152)) == 1     # 1152 = 9 x 128


def test_mfma_row_split_mirrors_the_native_choice():
    """Row-major 256x256 plans whose partial last tile row would add a round
    of tiles run their whole tiles first and the other rows on 128x128 tiles.
    The plan mirror names the same rows as the library: the workspace
    vt_gemm_check reports is the remainder's K-split partial sums, and the
    workgroups are both launches'."""
    from veritac_amd import _lib
    cases = {
        (1100, 14336, 4096, 1): (1024, 76, 1),     # 224 + 56 tiles: 1 round -> 2
        (2100, 8192, 1024, 1): (2048, 52, 1),      # 256 + 32; 52 rows on 128 64x64 tiles
        (4136, 4096, 1024, 1): (4096, 40, 2),      # 256 + 16; 40 rows on 64 64x64 tiles, K in 2
        (100, 14336, 4096, 11): (1024, 76, 1),     # 11 shared-B batches folded to 1100 rows
        (8000, 8192, 8192, 1): None,               # 992 and 1024 tiles: 4 rounds either way
        (2000, 8192, 4096, 1): None,               # 224 and 256: one round
        (300, 512, 256, 1): None,
        (8192, 8192, 8192, 1): None,               # whole tiles
        (1100, 14096, 4096, 1): None,              # N not whole tiles: one launch
    }
    for (m, n, k, batch), want in cases.items():
        plan = hg.make_plan(m, n, k, batch=batch, b_shared=batch > 1, variant="mfma_256x256")
        st, _, v, ks, ws = _lib.gemm_check(m, n, k, k, n, n, n, batch=batch,
                                           stride_a=m * k if batch > 1 else 0,
                                           stride_c=m * n if batch > 1 else 0,
                                           variant="mfma_256x256")
        assert st == _lib.VT_OK and v == "mfma_256x256" and ks == 0, (m, n, k)
        parts = hg._mfma_parts(plan)
        if want is None:
            assert parts is None and hg.mfma_split_rows(plan) == 0 and ws == 0, (m, n, k)
            continue
        top, rest = parts
        assert (top["m"], rest["m"], hg.mfma_k_split(rest)) == want, (m, n, k)
        assert rest["variant"] == "mfma_128x128" and top["batch"] == rest["batch"] == 1
        assert ws == (4 * want[2] * want[1] * n if want[2] > 1 else 0), (m, n, k)
        rows, cols = hg.mfma_tile_shape(rest)
        wgs = min(top["m"] // 256 * (n // 256), 256) + -(-rest["m"] // rows) * -(-n // cols) * want[2]
        assert hg.required_resources(plan) == (hg.persistent_lds(k), wgs)
        assert "%d rows on the persistent 256x256 kernel" % top["m"] in hg.native_check(plan)[1]
        # both launches priced, the first at whole tiles only
        t = hg.modeled_objective(plan, hg.modeled_counts(plan))[0]
        assert t == pytest.approx(sum(hg.modeled_objective(p, hg.modeled_counts(p))[0]
                                      for p in parts))
    # the 128x128 and 256x128 variants never split
    assert hg._mfma_parts(hg.make_plan(1100, 14336, 4096, variant="mfma_128x128")) is None


def test_mfma_selection_follows_the_measured_sweep():
    """The automatic choice among the MFMA tile shapes, on shapes whose three
    variants were timed on the GPU: the measured fastest (ties within 1 % take
    either). Moving a threshold of select_variant fails here. 256x128 tiles
    (M >= 256, N >= 128, K % 256 == 0; the last ones moved back when M or N
    is ragged) run on the persistent kernel's 256x128 form."""
    from veritac_amd import _lib
    either = ("mfma_128x128", "mfma_256x128")
    fastest = {
        (1024, 4096, 4096): "mfma_128x128", (1536, 4096, 4096): "mfma_256x128",
        (1536, 4096, 8192): "mfma_256x128", (2048, 4096, 4096): "mfma_256x128",
        (2560, 4096, 4096): "mfma_256x256", (3584, 4096, 4096): "mfma_256x256",
        (2560, 4096, 2048): "mfma_256x256", (768, 14336, 4096): "mfma_256x256",
        (9000, 1024, 4096): "mfma_256x256", (2048, 4096, 1024): either,
        (1536, 8192, 1024): "mfma_128x128", (1024, 14336, 1024): "mfma_256x256",
        (768, 14336, 512): "mfma_128x128", (9000, 1024, 512): "mfma_128x128",
        (3584, 4096, 256): "mfma_128x128", (600, 28672, 4096): "mfma_256x256",
        (8192, 8192, 8192): "mfma_256x256", (8000, 8192, 8192): "mfma_256x256",
        (1280, 4096, 1024): "mfma_256x128", (1280, 4096, 4096): "mfma_256x128",
        (2560, 2048, 2048): "mfma_256x128", (2560, 2048, 8192): "mfma_256x128",
        (768, 8192, 2048): "mfma_256x128", (512, 14336, 2048): "mfma_256x128",
        (1024, 8192, 1024): either, (2048, 2048, 4096): "mfma_128x128",
        (1280, 2048, 16384): "mfma_256x256", (768, 4096, 12288): "mfma_256x256",
        (512, 8192, 16384): "mfma_256x256", (2048, 4096, 32768): "mfma_256x256",
        (2048, 4096, 16384): either, (768, 2048, 16384): "mfma_256x128",
        (1024, 2048, 32768): "mfma_256x128", (512, 2048, 16384): "mfma_128x128",
        (1200, 4096, 1024): "mfma_256x128", (500, 14336, 2048): "mfma_256x128",
        (1800, 2048, 2048): "mfma_128x128", (2000, 4096, 4096): "mfma_256x128",
        (3000, 4096, 4096): "mfma_256x256",
    }
    for (m, n, k), want in fastest.items():
        want = (want,) if isinstance(want, str) else want
        assert _lib.select_variant(m, n, k, 1)[0] in want, (m, n, k)
        assert hg.make_plan(m, n, k)["variant"] in want, (m, n, k)


def test_mfma_column_split_mirrors_the_native_choice():
    """The column counterpart: whole 256-column tiles first when M is whole
    tiles and the partial tile column would add a round; the plan mirror
    names the same columns, remainder K split and workspace as the library."""
    from veritac_amd import _lib
    cases = {(8192, 8208, 8192): (8192, 16, 4), (4096, 4112, 4096): (4096, 16, 4),
             (4096, 4112, 1024): (4096, 16, 2), (2048, 4112, 1024): None,
             (8192, 8448, 8192): None, (8200, 8208, 8192): None}
    for (m, n, k), want in cases.items():
        plan = hg.make_plan(m, n, k, variant="mfma_256x256")
        st, _, v, ks, ws = _lib.gemm_check(m, n, k, k, n, n, n, variant="mfma_256x256")
        assert st == _lib.VT_OK and v == "mfma_256x256", (m, n, k)
        if want is None:
            assert hg.mfma_split_cols(plan) == 0, (m, n, k)
            continue
        top, rest = hg._mfma_parts(plan)
        assert (top["n"], rest["n"], hg.mfma_k_split(rest)) == want, (m, n, k)
        assert top["m"] == rest["m"] == m and rest["variant"] == "mfma_128x128"
        assert ws == 4 * want[2] * m * want[1], (m, n, k)
        # the remainder's 128x128 workgroups, or 64-row ones on a small grid
        # (16 columns: one tile column whatever its width)
        rows = hg.mfma_tile_shape(rest)[0]
        assert hg.required_resources(plan) == (
            hg.DMA16_LDS, min((m // 256) * (want[0] // 256), 256) + (m // rows) * want[2])
        assert "%d columns on the persistent 256x256 kernel" % want[0] in hg.native_check(plan)[1]


def test_small_128x128_grids_run_smaller_tiles():
    """mfma_128x128 with row-major B runs 64x128 tiles, with the K split those
    tiles call for, when that gives at most 256 workgroups, each over at most
    2048 of K (1024 per slice when K is split), and 64x64 tiles when they, with
    their own K split, meet the same bounds; packed B and other grids keep
    128x128 tiles. The native library reports the same K split (vt_gemm_check)."""
    from veritac_amd import _lib

    def tiles(m, n, k, **kw):
        plan = hg.make_plan(m, n, k, variant="mfma_128x128", **kw)
        return hg.mfma_tile_shape(plan), hg.mfma_k_split(plan), hg.required_resources(plan)
    quarter, half, full = (64, 64), (64, 128), (128, 128)
    q_lds, h_lds, f_lds = 3 * (64 * 64 + 64 * 64), 3 * (64 * 64 + 64 * 128), 3 * (128 * 64 + 64 * 128)
    assert (q_lds, h_lds) == (hg.QUARTER_TILE_LDS, hg.HALF_TILE_LDS)
    assert tiles(256, 256, 256, has_d=True, d_max_abs=1) == (quarter, 1, (q_lds, 16))
    assert tiles(1024, 1024, 1024) == (quarter, 1, (q_lds, 256))
    assert tiles(1024, 1024, 2048) == (quarter, 1, (q_lds, 256))
    assert tiles(512, 512, 2048) == (quarter, 4, (q_lds, 256))      # 64 tiles in 4 K slices
    assert tiles(1024, 2048, 512) == (half, 1, (h_lds, 256))        # 512 64x64 workgroups
    assert tiles(128, 4096, 4096) == (half, 4, (h_lds, 256))        # 64x64: K 4096 unsplit
    assert tiles(128, 1024, 16384) == (half, 16, (h_lds, 256))      # 64x64: 8 slices of 2048
    assert tiles(1152, 2048, 512) == (full, 1, (f_lds, 144))        # 288 64x128 workgroups
    assert tiles(2048, 2048, 512) == (full, 1, (f_lds, 256))
    assert tiles(256, 4096, 4096) == (full, 4, (f_lds, 256))        # 64x128: K 4096 unsplit
    assert tiles(128, 4096, 8192) == (full, 8, (f_lds, 256))        # 64x128: 4 slices of 2048
    assert tiles(512, 512, 256, batch=4) == (quarter, 1, (q_lds, 256))
    assert tiles(512, 512, 256, batch=8) == (half, 1, (h_lds, 256))
    assert tiles(512, 512, 256, batch=16, b_shared=True)[0] == full   # folded: 512 workgroups
    for m, n, k in ((1024, 1024, 1024), (512, 512, 2048), (256, 4096, 4096), (384, 1024, 1024),
                    (128, 4096, 4096), (128, 4096, 8192), (128, 1024, 16384), (256, 256, 8192)):
        _, _, v, ks, _ = _lib.gemm_check(m, n, k, k, n, n, n, variant="mfma_128x128")
        assert max(ks, 1) == hg.mfma_k_split(hg.make_plan(m, n, k, variant="mfma_128x128"))
    packed = hg._packed_parts(hg.make_plan(300, 1024, 1024, variant=hg.PACKED_VARIANT))[1]
    assert packed["variant"] == "mfma_128x128" and hg.mfma_tile_shape(packed) == full

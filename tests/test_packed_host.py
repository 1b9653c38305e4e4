"""Packed-B layout on the CPU: the oracle restatement is pinned by the GEMM it
must preserve (round trip, and the product read under the MFMA operand
convention equals A @ B), planted layout mistakes fail those checks, the
library's size query agrees, and the backend refuses mismatched operands
before any device call."""
import numpy as np
import pytest
import torch

from oracle import gemm_oracle as go
from oracle import packed_b as pk
from veritac_amd import HipGemmError, _lib
from veritac_amd.specializations.hip_gemm import backend as hg

SHAPES = [(1, 16), (16, 16), (64, 16), (100, 48), (130, 272), (256, 64), (1000, 32)]


def rand_b(k, n, seed):
    rng = np.random.default_rng(seed)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    B[0, :] = -128
    B[-1, ::2] = 127
    return B


@pytest.mark.parametrize("k,n", SHAPES)
def test_round_trip_and_size(k, n):
    B = rand_b(k, n, k * 131 + n)
    Bp = pk.pack_b(B)
    assert Bp.dtype == np.int8 and Bp.size == pk.packed_size(k, n) == n * (-(-k // 64) * 64)
    assert np.array_equal(pk.unpack_b(Bp, k, n), B)
    # padding rows contribute nothing: same multiset of nonzero bytes
    assert np.count_nonzero(Bp) == np.count_nonzero(B)
    assert int(np.abs(Bp.astype(np.int64)).sum()) == int(np.abs(B.astype(np.int64)).sum())


@pytest.mark.parametrize("k,n", SHAPES)
def test_packed_product_under_mfma_operand_convention(k, n):
    B = rand_b(k, n, 7 + k + n)
    A = np.random.default_rng(k).integers(-128, 128, (5, k), dtype=np.int8)
    assert np.array_equal(pk.gemm_from_packed(A, pk.pack_b(B), k, n), go.gemm_i8(A, B))


def _wrong_packs(B):
    """Plausible layout mistakes, each a full permutation of the right bytes."""
    k, n = B.shape
    kbt = -(-k // 64)
    pad = np.zeros((kbt * 64, n), np.int8)
    pad[:k] = B
    t = pad.reshape(kbt, 4, 16, n // 16, 16)
    yield "lane = column*4 + k group", t.transpose(3, 0, 4, 1, 2).reshape(-1)
    yield "tiles ordered [kb][nb]", t.transpose(0, 3, 1, 4, 2).reshape(-1)
    yield "tile bytes transposed", t.transpose(3, 0, 1, 2, 4).reshape(-1)


def test_planted_layout_mistakes_fail():
    k, n = 128, 48
    B = rand_b(k, n, 3)
    A = np.random.default_rng(4).integers(-128, 128, (4, k), dtype=np.int8)
    want = go.gemm_i8(A, B)
    for name, wrong in _wrong_packs(B):
        wrong = np.ascontiguousarray(wrong)
        assert not np.array_equal(pk.gemm_from_packed(A, wrong, k, n), want), name
        assert not np.array_equal(pk.unpack_b(wrong, k, n), B), name


def test_library_size_query_matches_layout():
    for k, n in SHAPES + [(0, 16), (4096, 14336), (4160, 14336)]:
        assert _lib.packed_b_size(k, n) == pk.packed_size(k, n)
    for k, n in [(64, 8), (64, 17), (-1, 16), (64, -16), (1 << 30, 16)]:
        with pytest.raises(HipGemmError):
            _lib.packed_b_size(k, n)


def test_packed_plans_validate():
    p = hg.make_plan(16, 14336, 4096, variant=hg.PACKED_VARIANT)
    assert hg.validate_plan(p) == (True, "ok")
    # 896 blocks: 224 whole groups of 4 blocks (8 half blocks)
    assert hg.packed_columns(p) == (8, 224)
    assert hg.required_resources(p) == (32768, 224)
    assert hg.packed_split(p) == (1, 64)
    # 2048 columns: 256 groups of one half block each, no K split
    p = hg.make_plan(40, 2048, 1024, variant=hg.PACKED_VARIANT)
    assert hg.packed_columns(p) == (1, 256) and hg.packed_split(p) == (1, 16)
    # few column groups: split K; up to 64 rows run in one group (row blocks
    # of 16); more rows on 128x128 tiles (one tile, K split in 2 slices of 512)
    p = hg.make_plan(40, 64, 1024, variant=hg.PACKED_VARIANT)
    assert hg.validate_plan(p)[0]
    assert hg.packed_columns(p) == (1, 8)
    assert hg.packed_split(p) == (2, 8)
    assert hg.required_resources(p)[1] == 8 * 2 * 1
    assert hg.required_resources(dict(p, m=100)) == (hg.TILES["mfma_128x128"][4], 2)
    # fewer than 192 whole groups: one group per CU, down to half a block;
    # at most 8 half blocks (4 tiles) per group; batches share the chip
    assert hg.packed_columns(dict(p, n=4800)) == (3, 200)
    assert hg.packed_columns(dict(p, n=8192)) == (4, 256)
    assert hg.packed_columns(dict(p, n=11200)) == (6, 234)
    assert hg.packed_columns(dict(p, n=12224)) == (6, 255)
    assert hg.packed_columns(dict(p, n=12272)) == (8, 192)
    assert hg.packed_columns(dict(p, n=4832)) == (3, 202)
    assert hg.packed_columns(dict(p, n=8208)) == (5, 206)
    assert hg.packed_columns(dict(p, n=4800, batch=2)) == (5, 120)
    assert hg.packed_columns(dict(p, n=16)) == (1, 2)
    for bad in (dict(n=24), dict(k=40), dict(batch=70000), dict(k_split=-1)):
        assert not hg.validate_plan(dict(p, **bad))[0], bad
    # packed is never an automatic candidate for a row-major B
    assert hg.PACKED_VARIANT not in hg.VARIANTS
    assert all(c["plan"]["variant"] != hg.PACKED_VARIANT
               for c in hg.optimize(16, 14336, 4096)["candidates"])


def test_packed_rows_in_whole_tiles_go_to_the_256_kernel():
    """Rows run on the 256x256 kernel when n % 256 == 0, k % 64 == 0 and there
    are at least 128 whole 256-row tiles: all of them, the last partial tile
    row moved back to end at m, unless that row adds a round of tiles on 256
    CUs; then the whole tiles, and more than 64 other rows on 128x128 tiles,
    up to 64 in one group on the decode kernel (the split vt_gemm_i8_packed
    makes in the library)."""
    plan = lambda m, n, k, **kw: hg.make_plan(m, n, k, variant=hg.PACKED_VARIANT, **kw)
    assert hg.PACKED_DMA_MIN_TILES == 128
    assert hg.packed_dma_rows(plan(8192, 8192, 8192)) == 8192
    assert hg.packed_dma_rows(plan(4096 + 44, 2048, 128)) == 4140     # 128 + 8 tiles: one round
    assert hg.packed_dma_rows(plan(4096 + 44, 2048, 128, batch=2)) == 4096   # 256 + 16: two
    assert hg.packed_dma_rows(plan(4096 + 44, 1792, 128)) == 0        # 16 x 7 = 112 tiles
    assert hg.packed_dma_rows(plan(768, 14336, 4096)) == 768          # 3 x 56 tiles
    assert hg.packed_dma_rows(plan(512, 14336, 4096)) == 0            # 2 x 56 tiles
    assert hg.packed_dma_rows(plan(256, 4096, 128, batch=8)) == 256   # 1 x 16 x 8 batches
    assert hg.packed_dma_rows(plan(300, 512, 128)) == 0               # 2 tiles
    assert hg.packed_dma_rows(plan(4096, 4352, 80)) == 0              # k not whole 64 slices
    # 16 column blocks of kbt 1 KiB tiles must stay within 32-bit lane offsets
    assert hg.packed_dma_rows(plan(256 * 128, 256, 64 * 262143)) == 256 * 128
    assert hg.packed_dma_rows(plan(256 * 128, 256, 64 * 262144)) == 0
    p = plan(4096 + 44, 2048, 128)
    assert hg.required_resources(p) == (hg.DMA_LDS, 136)
    assert "(4140 rows on the 256x256 kernel)" in hg.native_check(p)[1]
    p = plan(4096 + 44, 2048, 128, batch=2)
    assert hg.required_resources(p) == (hg.DMA_LDS, 256 + 2 * hg.packed_columns(dict(p, m=44))[1])
    assert "4096 rows on the 256x256 kernel, 44 in a group of up to 64" in hg.native_check(p)[1]
    p = plan(4096 + 100, 2048, 128, batch=2)
    assert hg.required_resources(p) == (hg.DMA_LDS, 256 + 2 * 16)
    assert "4096 rows on the 256x256 kernel, 100 on 128x128 tiles" in hg.native_check(p)[1]
    p = plan(300, 512, 128)
    assert hg.required_resources(p) == (hg.TILES["mfma_128x128"][4], 3 * 4)
    assert "300 on 128x128 tiles" in hg.native_check(p)[1]
    # a batch of rows after the 256-row tiles is not folded into one GEMM
    dma, rest = hg._packed_parts(plan(4096 + 100, 2048, 1024, batch=2, b_shared=True))
    assert dma["m"] == 4096 and rest["variant"] == "mfma_128x128" and not rest["b_shared"]
    # 8192^3 packed is modeled as the 256x256 kernel, not as 512 row groups
    big = plan(8192, 8192, 8192)
    t_packed = hg.modeled_objective(big, hg.modeled_counts(big))[0]
    row = hg.make_plan(8192, 8192, 8192, variant="mfma_256x256")
    assert t_packed == pytest.approx(hg.modeled_objective(row, hg.modeled_counts(row))[0])
    # 512 x 14336 x 4096 packed (224 tiles of 256x128) runs whole on the
    # persistent 256x128 form and is modeled as the row-major plan on it
    mid = plan(512, 14336, 4096)
    assert hg.packed_dma128(mid)
    row = hg.make_plan(512, 14336, 4096, variant="mfma_256x128")
    assert hg.modeled_objective(mid, hg.modeled_counts(mid)) == pytest.approx(
        hg.modeled_objective(row, hg.modeled_counts(row)))
    assert hg.required_resources(mid) == (hg.DMA16_LDS, 224)
    assert "512 rows on the 256x128 persistent kernel" in hg.native_check(mid)[1]
    # 128 such tiles or fewer, K below 1024 or N not whole 128-column tiles:
    # the routes above
    for m, n, k in ((1024, 4096, 4096), (1536, 4096, 512), (1536, 4000, 4096), (200, 14336, 4096)):
        assert not hg.packed_dma128(plan(m, n, k)), (m, n, k)
    assert hg.packed_dma128(plan(2000, 4096, 4096))          # ragged M: last tile row moved back


def test_run_refuses_mismatched_packed_operands():
    calls = []

    def fake(plan, A, B, D, C, stream):
        calls.append(plan["variant"])

    k, n = 128, 64
    A = torch.zeros((16, k), dtype=torch.int8)
    B = torch.zeros((k, n), dtype=torch.int8)
    Bp = hg.PackedB(torch.zeros(pk.packed_size(k, n), dtype=torch.int8), k, n)
    plan = hg.make_plan(16, n, k, variant=hg.PACKED_VARIANT)
    hg.run(plan, A, Bp, runner=fake)
    assert calls == [hg.PACKED_VARIANT]
    with pytest.raises(HipGemmError, match="packed by pack_b"):
        hg.run(plan, A, B, runner=fake)
    with pytest.raises(HipGemmError, match="needs variant"):
        hg.run(hg.make_plan(16, n, k, variant="skinny"), A, Bp, runner=fake)
    with pytest.raises(HipGemmError, match="plan needs"):
        hg.run(hg.make_plan(16, n + 16, k, variant=hg.PACKED_VARIANT), A[:, :k],
               Bp, runner=fake)
    short = hg.PackedB(torch.zeros(100, dtype=torch.int8), k, n)
    with pytest.raises(HipGemmError, match="contiguous int8"):
        hg.run(plan, A, short, runner=fake)
    assert calls == [hg.PACKED_VARIANT]


def test_pack_b_refuses_host_tensors():
    with pytest.raises(HipGemmError, match="no CPU path"):
        hg.pack_b(torch.zeros((64, 16), dtype=torch.int8))
    with pytest.raises(HipGemmError):
        hg.pack_b(torch.zeros((64, 16), dtype=torch.int32))

"""Packed-B decode path on the GPU, through the C ABI (needs a gfx950 GPU).

vt_pack_b_i8 must produce the oracle's packed bytes exactly, and
vt_gemm_i8_packed must give C = D + A.B bit for bit: the same result as the
oracle and as vt_gemm_i8 on the row-major B. Outputs are poisoned with
INT32_MIN before each launch so unwritten cells show.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import gemm_oracle as go
from oracle import packed_b as pk
from veritac_amd import HipGemmError, _lib
from veritac_amd.specializations.hip_gemm import backend as hg
from veritac_amd.specializations.hip_gemm import inputs

pytestmark = pytest.mark.gpu

INT32_MIN = -2**31


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    assert _lib.load_library().vt_device_count() >= 1, "GPU visible but not gfx950"
    return torch.device("cuda", 0)


def say(*args):
    print(*args, flush=True)


def to_dev(dev, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def gpu_pack(dev, B, ldb=None):
    """vt_pack_b_i8 of a row-major B (optionally with a padded row pitch)."""
    k, n = B.shape
    ldb = n if ldb is None else ldb
    host = np.zeros((k, ldb), np.int8)
    host[:, :n] = B
    Bt = to_dev(dev, host)
    size = _lib.packed_b_size(k, n)
    Bp = torch.full((max(size, 16),), 0x5A, dtype=torch.int8, device=dev)
    _lib.pack_b_raw(Bt.data_ptr(), Bp.data_ptr(), k, n, ldb)
    _lib.sync(None)
    return Bp[:size].cpu().numpy()


def gpu_gemm_packed(dev, A, B, D=None, k_split=0, in_place=False):
    """Pack B on the GPU, then C = D + A.B through vt_gemm_i8_packed."""
    M, K = A.shape
    N = B.shape[1]
    Bt = to_dev(dev, B)
    size = _lib.packed_b_size(K, N)
    Bp = torch.empty(size, dtype=torch.int8, device=dev)
    _lib.pack_b_raw(Bt.data_ptr(), Bp.data_ptr(), K, N, N)
    At = to_dev(dev, A)
    if in_place:
        C = to_dev(dev, D)
        Dt = C
    else:
        C = torch.full((M, N), INT32_MIN, dtype=torch.int32, device=dev)
        Dt = to_dev(dev, D) if D is not None else None
    _lib.gemm_packed_raw(At.data_ptr(), Bp.data_ptr(), Dt.data_ptr() if Dt is not None else None,
                         C.data_ptr(), M, N, K, K, N, N, k_split=k_split)
    _lib.sync(None)
    return C.cpu().numpy()


@pytest.mark.parametrize("k,n", [(1, 16), (64, 16), (100, 48), (130, 272), (4096, 256),
                                 (1000, 14336)])
def test_pack_matches_oracle_bytes(dev, k, n):
    say("pack", k, n)
    B = np.random.default_rng(k + n).integers(-128, 128, (k, n), dtype=np.int8)
    assert np.array_equal(gpu_pack(dev, B), pk.pack_b(B))


def test_pack_with_row_pitch_and_batches(dev):
    k, n, batch, ldb = 200, 80, 3, 112
    rng = np.random.default_rng(9)
    B = rng.integers(-128, 128, (batch, k, ldb), dtype=np.int8)
    Bt = to_dev(dev, B)
    size = _lib.packed_b_size(k, n)
    stride_bp = size + 1024
    Bp = torch.full((batch * stride_bp,), 0x33, dtype=torch.int8, device=dev)
    _lib.pack_b_raw(Bt.data_ptr(), Bp.data_ptr(), k, n, ldb, batch, k * ldb, stride_bp)
    _lib.sync(None)
    got = Bp.cpu().numpy()
    for b in range(batch):
        part = got[b * stride_bp:(b + 1) * stride_bp]
        assert np.array_equal(part[:size], pk.pack_b(B[b, :, :n])), b
        assert np.all(part[size:] == 0x33), b   # nothing written past the packed size


def test_full_packed_config4_full_output(dev):
    """Config 4 (M = 1 and 16, K = 4096, N = 14336) through pack_b / run."""
    for m in (16, 1):
        c = inputs.config_inputs(4, seed=0, m=m)
        say("config 4 packed m=%d" % m)
        A, B = to_dev(dev, c["A"]), to_dev(dev, c["B"])
        Bp = hg.pack_b(B)
        plan = hg.make_plan(m, 14336, 4096, variant=hg.PACKED_VARIANT)
        C = hg.run(plan, A, Bp).cpu().numpy()
        assert np.array_equal(C, go.gemm_i8_f64(c["A"], c["B"])), m
        C_row = hg.run(hg.make_plan(m, 14336, 4096), A, B).cpu().numpy()
        assert np.array_equal(C, C_row), m


@pytest.mark.parametrize("m,k,n", [(1, 16, 16), (3, 48, 80), (16, 64, 64), (16, 80, 48),
                                   (7, 4160, 272), (16, 1024, 2048), (17, 256, 128),
                                   (40, 512, 96), (5, 8192, 32)])
@pytest.mark.parametrize("k_split", [0, 1, 3])
def test_edge_shapes_and_splits(dev, m, k, n, k_split):
    say("packed", m, k, n, "k_split", k_split)
    rng = np.random.default_rng(m * 1000 + k + n + k_split)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    assert np.array_equal(gpu_gemm_packed(dev, A, B, k_split=k_split), go.gemm_i8(A, B))


@pytest.mark.parametrize("k_split", [0, 1, 4])
def test_initial_partial_sum_and_in_place(dev, k_split):
    rng = np.random.default_rng(5 + k_split)
    m, k, n = 16, 2048, 1024
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = rng.integers(-2**20, 2**20, (m, n), dtype=np.int32)
    want = go.gemm_i8(A, B, D)
    assert np.array_equal(gpu_gemm_packed(dev, A, B, D, k_split=k_split), want)
    assert np.array_equal(gpu_gemm_packed(dev, A, B, D, k_split=k_split, in_place=True), want)


def test_extremes_at_k8192(dev):
    m, k, n = 16, 8192, 64
    A = np.full((m, k), -128, np.int8)
    B = np.full((k, n), -128, np.int8)
    C = gpu_gemm_packed(dev, A, B)
    assert np.all(C == 134217728)
    A = np.tile(np.array([-128, 127], np.int8), (m, k // 2))
    B = np.tile(np.array([[127], [-128]], np.int8), (k // 2, n))
    assert np.array_equal(gpu_gemm_packed(dev, A, B), go.gemm_i8(A, B))


@pytest.mark.parametrize("shared", [True, False])
def test_batches(dev, shared):
    rng = np.random.default_rng(11 + shared)
    batch, m, k, n = 3, 16, 512, 192
    A = rng.integers(-128, 128, (batch, m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n) if shared else (batch, k, n), dtype=np.int8)
    D = rng.integers(-1000, 1000, (batch, m, n), dtype=np.int32)
    At, Bt, Dt = to_dev(dev, A), to_dev(dev, B), to_dev(dev, D)
    Bp = hg.pack_b(Bt)
    plan = hg.make_plan(m, n, k, batch=batch, b_shared=shared, has_d=True, d_max_abs=1000,
                        variant=hg.PACKED_VARIANT)
    C = hg.run(plan, At, Bp, Dt).cpu().numpy()
    for b in range(batch):
        Bb = B if shared else B[b]
        assert np.array_equal(C[b], go.gemm_i8(A[b], Bb, D[b])), b


def test_repeated_launches_stay_exact(dev):
    c = inputs.config_inputs(4, seed=3, m=16)
    A, B = to_dev(dev, c["A"]), to_dev(dev, c["B"])
    Bp = hg.pack_b(B)
    plan = hg.make_plan(16, 14336, 4096, variant=hg.PACKED_VARIANT)
    want = go.gemm_i8_f64(c["A"], c["B"])
    outs = [torch.full((16, 14336), INT32_MIN, dtype=torch.int32, device=dev) for _ in range(4)]
    for i in range(20):
        hg.run(plan, A, Bp, out=outs[i % 4])
    torch.cuda.synchronize()
    for C in outs:
        assert np.array_equal(C.cpu().numpy(), want)


def test_refusals_never_launch(dev):
    A = torch.zeros((16, 64), dtype=torch.int8, device=dev)
    Bp = torch.zeros(64 * 64, dtype=torch.int8, device=dev)
    C = torch.zeros((16, 64), dtype=torch.int32, device=dev)
    with pytest.raises(HipGemmError):   # N not a multiple of 16
        _lib.gemm_packed_raw(A.data_ptr(), Bp.data_ptr(), None, C.data_ptr(), 16, 40, 64, 64, 40, 64)
    with pytest.raises(HipGemmError):   # K not a multiple of 16
        _lib.gemm_packed_raw(A.data_ptr(), Bp.data_ptr(), None, C.data_ptr(), 16, 64, 40, 64, 64, 64)
    with pytest.raises(HipGemmError):   # misaligned A
        _lib.gemm_packed_raw(A.data_ptr() + 1, Bp.data_ptr(), None, C.data_ptr(), 16, 64, 64, 64,
                             64, 64)
    with pytest.raises(HipGemmError):   # ldc < N
        _lib.gemm_packed_raw(A.data_ptr(), Bp.data_ptr(), None, C.data_ptr(), 16, 64, 64, 64, 64, 32)
    with pytest.raises(HipGemmError):   # pack: ldb < N
        _lib.pack_b_raw(A.data_ptr(), Bp.data_ptr(), 16, 64, 48)
    _lib.sync(None)


def test_repack_in_place(dev):
    rng = np.random.default_rng(21)
    k, n = 320, 96
    B1 = rng.integers(-128, 128, (k, n), dtype=np.int8)
    B2 = rng.integers(-128, 128, (k, n), dtype=np.int8)
    Bp = hg.pack_b(to_dev(dev, B1))
    same = hg.pack_b(to_dev(dev, B2), out=Bp)
    assert same is Bp
    assert np.array_equal(Bp.data.cpu().numpy(), pk.pack_b(B2))
    with pytest.raises(HipGemmError, match="out must be"):
        hg.pack_b(to_dev(dev, B2[:, :80]), out=Bp)


# N -> (8-column half blocks per group, groups) on a 256-CU MI355X (packed_columns):
# 400 -> (1, 50): every group is half a block; 3200 -> (2, 200); 4832 -> (3, 202):
# the last group is the upper half of the last block; 6400 -> (4, 200);
# 8208 -> (5, 206): last group again an upper half; 11200 -> (6, 234): last group
# one block; 11600 -> (6, 242); 12224 -> (6, 255); 13600 -> (8, 213): whole
# groups, the last one two blocks; 17600 -> (8, 275): two rounds of the CUs
HALF_BLOCK_NS = [400, 3200, 4832, 6400, 8208, 11200, 11600, 12224, 13600, 17600]


@pytest.mark.parametrize("n", HALF_BLOCK_NS)
@pytest.mark.parametrize("m", [1, 16])
def test_half_block_column_groups_write_every_column_once(dev, m, n):
    """Column groups that start or end on half a 16-column block: C starts as
    D (added in place) and every cell must equal D + A.B."""
    k = 320
    plan = hg.make_plan(m, n, k, has_d=True, d_max_abs=1 << 20, variant=hg.PACKED_VARIANT)
    hpw, groups = hg.packed_columns(plan)
    say("half blocks", m, n, "hpw", hpw, "groups", groups)
    assert hg.packed_split(plan)[0] == 1          # K = 320: one slice per wave at most
    rng = np.random.default_rng(n + m)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = rng.integers(-2**20, 2**20, (m, n), dtype=np.int32)
    Dt = to_dev(dev, D)
    C = hg.run(plan, to_dev(dev, A), hg.pack_b(to_dev(dev, B)), Dt, out=Dt)
    assert np.array_equal(C.cpu().numpy(), go.gemm_i8(A, B, D))


def test_half_block_groups_across_batches(dev):
    batch, m, k, n = 2, 16, 256, 4800          # 1200 half blocks -> 5 per group, 240 groups
    plan = hg.make_plan(m, n, k, batch=batch, variant=hg.PACKED_VARIANT)
    assert hg.packed_columns(plan) == (5, 120)
    rng = np.random.default_rng(2)
    A = rng.integers(-128, 128, (batch, m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (batch, k, n), dtype=np.int8)
    out = torch.full((batch, m, n), INT32_MIN, dtype=torch.int32, device=dev)
    C = hg.run(plan, to_dev(dev, A), hg.pack_b(to_dev(dev, B)), out=out).cpu().numpy()
    for b in range(batch):
        assert np.array_equal(C[b], go.gemm_i8(A[b], B[b])), b


# Packed rows take one of three kernels: whole 256-row tiles on the persistent
# 256x256 DMA kernel when N % 256 == 0, K % 64 == 0 and there are at least
# 128 of them; more than 64 other rows on 128x128 tiles (K split when the grid
# is small); up to 64 rows in a group on the decode kernel.
@pytest.mark.parametrize("m,k,n", [(256, 64, 256), (512, 192, 768), (300, 128, 512),
                                   (1024, 1024, 1024), (768, 4160, 256)])
def test_tile_rows_with_packed_b(dev, m, k, n):
    say("packed tiles", m, k, n)
    rng = np.random.default_rng(m + 7 * k + n)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    assert np.array_equal(gpu_gemm_packed(dev, A, B), go.gemm_i8_f64(A, B))


def test_tile_rows_with_packed_b_d_in_place(dev):
    m, k, n = 768, 512, 512
    rng = np.random.default_rng(31)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = rng.integers(-2**30, 2**30, (m, n), dtype=np.int32)
    want = go.gemm_i8(A, B, D)
    assert np.array_equal(gpu_gemm_packed(dev, A, B, D), want)
    assert np.array_equal(gpu_gemm_packed(dev, A, B, D, in_place=True), want)


def test_tile_rows_with_packed_b_extremes(dev):
    m, k, n = 256, 8192, 256
    A = np.full((m, k), -128, np.int8)
    B = np.full((k, n), -128, np.int8)
    assert np.all(gpu_gemm_packed(dev, A, B) == 134217728)
    A = np.tile(np.array([-128, 127], np.int8), (m, k // 2))
    B = np.tile(np.array([[127], [-128]], np.int8), (k // 2, n))
    assert np.array_equal(gpu_gemm_packed(dev, A, B), go.gemm_i8_f64(A, B))


@pytest.mark.parametrize("shared", [True, False])
def test_tile_rows_with_packed_b_batches(dev, shared):
    rng = np.random.default_rng(41 + shared)
    batch, m, k, n = 3, 272, 256, 512        # 128x128 tiles; shared B folds the batches
    A = rng.integers(-128, 128, (batch, m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n) if shared else (batch, k, n), dtype=np.int8)
    D = rng.integers(-1000, 1000, (batch, m, n), dtype=np.int32)
    At, Bt, Dt = to_dev(dev, A), to_dev(dev, B), to_dev(dev, D)
    plan = hg.make_plan(m, n, k, batch=batch, b_shared=shared, has_d=True, d_max_abs=1000,
                        variant=hg.PACKED_VARIANT)
    C = hg.run(plan, At, hg.pack_b(Bt), Dt).cpu().numpy()
    for b in range(batch):
        Bb = B if shared else B[b]
        assert np.array_equal(C[b], go.gemm_i8(A[b], Bb, D[b])), b


def test_tile_rows_with_packed_b_equal_row_major_config5_shape(dev):
    """2048^3 on config-5-like data: packed B and row-major B give the same
    full output, which equals the exact float64 product."""
    n = 2048
    c = inputs.config_inputs(5, seed=4)
    A, B = c["A"][:n, :n].copy(), c["B"][:n, :n].copy()
    At, Bt = to_dev(dev, A), to_dev(dev, B)
    plan_p = hg.make_plan(n, n, n, variant=hg.PACKED_VARIANT)
    Cp = hg.run(plan_p, At, hg.pack_b(Bt)).cpu().numpy()
    Cr = hg.run(hg.make_plan(n, n, n, variant="mfma_256x256"), At, Bt).cpu().numpy()
    assert np.array_equal(Cp, Cr)
    assert np.array_equal(Cp, go.gemm_i8_f64(A, B))


# Up to 64 rows run as 1, 2 or 4 row blocks of 16 over one stream of packed B;
# more rows as groups of 64.
@pytest.mark.parametrize("m", [17, 32, 33, 48, 64, 100, 130])
@pytest.mark.parametrize("k_split", [0, 3])
def test_row_blocks_with_packed_b(dev, m, k_split):
    rng = np.random.default_rng(1000 + m + k_split)
    k, n = 1088, 4800        # 4800 columns: half-block column groups (masked)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = rng.integers(-2**20, 2**20, (m, n), dtype=np.int32)
    say("packed row blocks", m, "k_split", k_split)
    assert np.array_equal(gpu_gemm_packed(dev, A, B, k_split=k_split), go.gemm_i8(A, B))
    assert np.array_equal(gpu_gemm_packed(dev, A, B, D, k_split=k_split, in_place=True),
                          go.gemm_i8(A, B, D))


def test_row_blocks_with_packed_b_whole_groups(dev):
    """N = 14336: whole column groups (unmasked), 64 rows, extremes at K = 4096."""
    m, k, n = 64, 4096, 14336
    A = np.tile(np.array([-128, 127], np.int8), (m, k // 2))
    B = np.tile(np.array([[127], [-128]], np.int8), (k // 2, n))
    assert np.array_equal(gpu_gemm_packed(dev, A, B), go.gemm_i8_f64(A, B))
    c = inputs.config_inputs(4, seed=2, m=16)
    A = np.concatenate([c["A"]] * 4)          # 64 rows
    assert np.array_equal(gpu_gemm_packed(dev, A, c["B"]), go.gemm_i8_f64(A, c["B"]))


# 128x128 tiles with packed B: K tails (K % 128 == 64, K % 64 == 16, K of one
# zero-padded 64-row block), ragged N (last 128-column tile partly live), K
# split into 2 and 16 slices, D in place.
@pytest.mark.parametrize("m,k,n", [(65, 4160, 272), (100, 1040, 400), (200, 1024, 64),
                                   (128, 16384, 1024), (129, 2048, 4096), (100, 16, 48),
                                   (130, 48, 80)])
def test_packed_tiles_edges_and_k_split(dev, m, k, n):
    plan = hg.make_plan(m, n, k, variant=hg.PACKED_VARIANT)
    say("packed tiles", m, k, n, hg.native_check(plan)[1])
    rng = np.random.default_rng(7 * m + k + n)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = rng.integers(-2**30, 2**30, (m, n), dtype=np.int32)
    assert np.array_equal(gpu_gemm_packed(dev, A, B), go.gemm_i8(A, B))
    assert np.array_equal(gpu_gemm_packed(dev, A, B, D, in_place=True), go.gemm_i8(A, B, D))


def test_packed_tiles_k_split_extremes(dev):
    """128 x 1024 x 16384 (16 K slices) on constant extremes: every partial sum
    and the reduction at their largest magnitudes."""
    m, k, n = 128, 16384, 1024
    A = np.full((m, k), -128, np.int8)
    B = np.full((k, n), -128, np.int8)
    assert np.all(gpu_gemm_packed(dev, A, B) == 268435456)
    A = np.tile(np.array([-128, 127], np.int8), (m, k // 2))
    B = np.tile(np.array([[127], [-128]], np.int8), (k // 2, n))
    assert np.array_equal(gpu_gemm_packed(dev, A, B), go.gemm_i8_f64(A, B))


@pytest.mark.parametrize("extra,k", [(0, 192), (44, 192), (100, 192), (0, 256), (100, 512)])
def test_dma_rows_with_packed_b(dev, extra, k):
    """4096 + extra rows x 2048 columns, all on the DMA kernel (32x32x32 at
    K = 192, 16x16x64 at K = 256 and 512): 128 whole 256-row tiles, and for
    44 or 100 extra rows a last tile row moved back to end at M (136 tiles,
    still one round), its stores masked; in place as well."""
    m, n = 4096 + extra, 2048
    plan = hg.make_plan(m, n, k, variant=hg.PACKED_VARIANT)
    assert hg.packed_dma_rows(plan) == m
    say("packed dma", m, k, n, hg.native_check(plan)[1])
    rng = np.random.default_rng(300 + extra + k)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = rng.integers(-2**20, 2**20, (m, n), dtype=np.int32)
    assert np.array_equal(gpu_gemm_packed(dev, A, B), go.gemm_i8_f64(A, B))
    assert np.array_equal(gpu_gemm_packed(dev, A, B, D, in_place=True), go.gemm_i8(A, B, D))


@pytest.mark.parametrize("shared", [True, False])
def test_dma_rows_with_packed_b_batches(dev, shared):
    """8 batches of 256 x 4096: 128 tiles over the batches on the DMA kernel."""
    rng = np.random.default_rng(51 + shared)
    batch, m, k, n = 8, 256, 128, 4096
    A = rng.integers(-128, 128, (batch, m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n) if shared else (batch, k, n), dtype=np.int8)
    D = rng.integers(-1000, 1000, (batch, m, n), dtype=np.int32)
    plan = hg.make_plan(m, n, k, batch=batch, b_shared=shared, has_d=True, d_max_abs=1000,
                        variant=hg.PACKED_VARIANT)
    assert hg.packed_dma_rows(plan) == 256
    At, Bt, Dt = to_dev(dev, A), to_dev(dev, B), to_dev(dev, D)
    C = hg.run(plan, At, hg.pack_b(Bt), Dt).cpu().numpy()
    for b in range(batch):
        Bb = B if shared else B[b]
        assert np.array_equal(C[b], go.gemm_i8(A[b], Bb, D[b])), b


@pytest.mark.parametrize("extra", [100, 44])
def test_packed_tiles_after_dma_rows_in_batches(dev, extra):
    """2 batches of 4096 + extra rows, shared packed B: 256 whole tiles plus
    16 partial ones would add a round, so the DMA kernel takes the whole
    tiles of both batches, then each batch's last rows run batch by batch
    (not folded: those rows are not contiguous), 100 on 128x128 tiles or 44
    in a decode group."""
    rng = np.random.default_rng(61 + extra)
    batch, m, k, n = 2, 4096 + extra, 128, 2048
    A = rng.integers(-128, 128, (batch, m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    plan = hg.make_plan(m, n, k, batch=batch, b_shared=True, variant=hg.PACKED_VARIANT)
    assert hg.packed_dma_rows(plan) == 4096
    At, Bt = to_dev(dev, A), to_dev(dev, B)
    C = hg.run(plan, At, hg.pack_b(Bt)).cpu().numpy()
    for b in range(batch):
        assert np.array_equal(C[b], go.gemm_i8_f64(A[b], B)), b


# m, n, k, explicit k_split (0: automatic), whether the slices finish in the
# kernel (finishing words) rather than in the reduction launch
PACKED_FINISH = [
    (1, 1024, 4096, 0, True),      # 128 half-block groups, K in 2 slices
    (3, 1024, 4096, 0, True),      # odd rows: the last word's second row is empty
    (16, 512, 4096, 0, True),      # K in 4 slices
    (16, 1024, 8192, 0, True),
    (8, 2048, 4096, 3, True),      # an explicit split
    (17, 1024, 4096, 0, False),    # two row blocks: the reduction launch
    (16, 14336, 4096, 0, False),   # whole groups, K unsplit
]


@pytest.mark.parametrize("m,n,k,ks,finishes", PACKED_FINISH)
def test_packed_k_slices_finished_in_the_kernel(dev, m, n, k, ks, finishes):
    """Packed-B decode launches that split K finish the slices in the kernel
    up to 16 rows, through the same finishing words as the row-major decode
    kernel; out of place, with D and in place (wrapping past int32)."""
    plan = hg.make_plan(m, n, k, variant=hg.PACKED_VARIANT, k_split=ks)
    assert hg.packed_finishes(plan) == finishes
    assert (hg.packed_split(plan)[0] > 1) == (finishes or m > 16)
    rng = np.random.default_rng(m * 7 + n + k)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = np.where(rng.integers(0, 2, (m, n)) == 1, 2**31 - 9, -2**31 + 9).astype(np.int32)
    say("packed finish", m, n, k, ks)
    assert np.array_equal(gpu_gemm_packed(dev, A, B, k_split=ks), go.gemm_i8(A, B, None))
    want = go.gemm_i8(A, B, D)
    assert np.array_equal(gpu_gemm_packed(dev, A, B, D, k_split=ks), want)
    assert np.array_equal(gpu_gemm_packed(dev, A, B, D, k_split=ks, in_place=True), want)


def test_packed_finish_repeated_and_mixed(dev):
    """Finishing and two-launch packed calls in turn on one stream, with the
    row-major decode's finishing calls between them: the words every call
    leaves zero serve the next."""
    rng = np.random.default_rng(77)
    for it, (m, n, k, packed) in enumerate(((2, 1024, 4096, True), (16, 1024, 4096, False),
                                            (17, 1024, 4096, True), (5, 512, 4096, True),
                                            (1, 2048, 2048, False), (16, 1024, 4096, True))):
        A = rng.integers(-128, 128, (m, k), dtype=np.int8)
        B = rng.integers(-128, 128, (k, n), dtype=np.int8)
        say("packed finish repeat", it, m, n, k, packed)
        if packed:
            got = gpu_gemm_packed(dev, A, B)
        else:
            At, Bt = to_dev(dev, A), to_dev(dev, B)
            got = hg.run(hg.make_plan(m, n, k), At, Bt).cpu().numpy()
        assert np.array_equal(got, go.gemm_i8(A, B, None)), it


# Packed B on the persistent kernel's 256x128 form (more than 128 but at most
# 256 tiles of 256x128, K >= 1024 in whole 256-deep groups, N in whole
# 128-column tiles): whole and ragged M, D out of place and in place.
@pytest.mark.parametrize("m,k,n", [(1536, 1024, 4096), (2000, 1024, 4096), (512, 2048, 14336),
                                   (1280, 1280, 4096)])
def test_packed_b_on_the_256x128_form(dev, m, k, n):
    plan = hg.make_plan(m, n, k, variant=hg.PACKED_VARIANT)
    assert hg.packed_dma128(plan)
    rng = np.random.default_rng(m + k + n)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = rng.integers(-2**20, 2**20, (m, n), dtype=np.int32)
    say("packed 256x128 form", m, k, n)
    assert np.array_equal(gpu_gemm_packed(dev, A, B), go.gemm_i8(A, B, None))
    want = go.gemm_i8(A, B, D)
    assert np.array_equal(gpu_gemm_packed(dev, A, B, D), want)
    assert np.array_equal(gpu_gemm_packed(dev, A, B, D, in_place=True), want)


@pytest.mark.parametrize("shared", [True, False])
def test_packed_b_on_the_256x128_form_batches(dev, shared):
    """Two batches of 768 x 4096 (192 tiles in all), one packed B for both or
    one each, with D."""
    rng = np.random.default_rng(77 + shared)
    batch, m, k, n = 2, 768, 1024, 4096
    A = rng.integers(-128, 128, (batch, m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n) if shared else (batch, k, n), dtype=np.int8)
    D = rng.integers(-1000, 1000, (batch, m, n), dtype=np.int32)
    plan = hg.make_plan(m, n, k, batch=batch, b_shared=shared, has_d=True, d_max_abs=1000,
                        variant=hg.PACKED_VARIANT)
    assert hg.packed_dma128(plan)
    say("packed 256x128 form batches", shared)
    C = hg.run(plan, to_dev(dev, A), hg.pack_b(to_dev(dev, B)), to_dev(dev, D)).cpu().numpy()
    for b in range(batch):
        assert np.array_equal(C[b], go.gemm_i8(A[b], B if shared else B[b], D[b])), b

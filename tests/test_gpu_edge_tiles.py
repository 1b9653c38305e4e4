"""Row-major problems whose M or N is not a whole number of 256 tiles on the
persistent 256x256 kernels (needs a gfx950 GPU), against the oracle through
the C ABI.

One launch takes them when M, N >= 256 and K is whole 64-deep slices: the
last tile row (column) starts at M - 256 (N - 256), so its loads stay inside
A and B, and it leaves the rows (columns) it shares with its neighbour to the
neighbour's stores, so every element is written once, in place as well. When
the partial tile row would add a round of tiles, the whole 256-row tiles run
first and the remaining rows on 128x128 tiles. Cases cover both kernels
(K % 256 == 0 on 16x16x64, other multiples of 64 on 32x32x32), D out of
place and in place, batches, the split with a K-split remainder, and that
nothing outside C's M x N block is written.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import gemm_oracle as go
from veritac_amd import _lib
from veritac_amd.specializations.hip_gemm import backend as hg

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


def operands(m, n, k, seed, batch=None, d_bound=2**30):
    rng = np.random.default_rng(seed)
    lead = () if batch is None else (batch,)
    A = rng.integers(-128, 128, lead + (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, lead + (k, n), dtype=np.int8)
    A.reshape(-1)[:k] = -128             # an extreme row and column
    B[..., :, 0] = -128
    D = rng.integers(-d_bound, d_bound, lead + (m, n), dtype=np.int32)
    return A, B, D


def gemm_padded(dev, A, B, D, ldc, extra_rows, in_place=False):
    """One vt_gemm_i8 call on mfma_256x256 with C inside a buffer of ldc
    columns and extra_rows more rows, all poisoned: returns (C, buffer)."""
    m, k = A.shape
    n = B.shape[1]
    At, Bt = to_dev(dev, A), to_dev(dev, B)
    buf = torch.full((m + extra_rows, ldc), INT32_MIN, dtype=torch.int32, device=dev)
    Dt, ldd = None, 0
    if D is not None and in_place:
        buf[:m, :n] = to_dev(dev, D)
        Dt, ldd = buf, ldc
    elif D is not None:
        Dt, ldd = to_dev(dev, D), n
    _lib.gemm_raw(At.data_ptr(), Bt.data_ptr(), Dt.data_ptr() if Dt is not None else None,
                  buf.data_ptr(), m, n, k, k, n, ldd, ldc, variant="mfma_256x256")
    _lib.sync(None)
    got = buf.cpu().numpy()
    return got[:m, :n], got


@pytest.mark.parametrize("m,n,k", [
    (300, 512, 256),      # M ragged, 16x16x64
    (256, 272, 1024),     # N ragged by 16 columns
    (520, 784, 2304),     # both, 16x16x64
    (700, 1040, 320),     # both, 32x32x32 (K % 256 != 0)
    (257, 257 + 15, 192),  # one row and 16 columns past a tile, 32x32x32
])
@pytest.mark.parametrize("with_d", [False, True])
def test_last_tiles_moved_back(dev, m, n, k, with_d):
    n = n // 16 * 16
    say("edge tiles", m, n, k, "D" if with_d else "")
    A, B, D = operands(m, n, k, m * 7 + n + k)
    want = go.gemm_i8(A, B, D) if with_d else go.gemm_i8_f64(A, B)
    C, buf = gemm_padded(dev, A, B, D if with_d else None, ldc=n + 4, extra_rows=3)
    assert np.array_equal(C, want)
    assert (buf[:m, n:] == INT32_MIN).all() and (buf[m:] == INT32_MIN).all()


@pytest.mark.parametrize("m,n,k", [(300, 512, 256), (520, 784, 2304), (700, 1040, 320)])
def test_in_place_on_ragged_tiles(dev, m, n, k):
    """C = C + A.B on moved-back tiles: the rows and columns a last tile
    shares with its neighbour are stored once, so no element adds D twice."""
    n = n // 16 * 16
    say("edge tiles in place", m, n, k)
    A, B, D = operands(m, n, k, m + n + k + 1)
    C, buf = gemm_padded(dev, A, B, D, ldc=n + 4, extra_rows=2, in_place=True)
    assert np.array_equal(C, go.gemm_i8(A, B, D))
    assert (buf[:m, n:] == INT32_MIN).all() and (buf[m:] == INT32_MIN).all()


@pytest.mark.parametrize("shared", [False, True])
def test_batches_with_ragged_rows(dev, shared):
    """Unshared B: each batch's last tile row moves back inside that batch.
    Shared B folds 3 x 100 rows into 300 stacked rows whose last tile spans
    the batch boundaries."""
    batch, m, n, k = 3, (100 if shared else 300), 512, 512
    rng = np.random.default_rng(41 + shared)
    A = rng.integers(-128, 128, (batch, m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n) if shared else (batch, k, n), dtype=np.int8)
    D = rng.integers(-1000, 1000, (batch, m, n), dtype=np.int32)
    plan = hg.make_plan(m, n, k, batch=batch, b_shared=shared, has_d=True, d_max_abs=1000,
                        variant="mfma_256x256")
    say("edge tiles batches", shared)
    C = hg.run(plan, to_dev(dev, A), to_dev(dev, B), to_dev(dev, D)).cpu().numpy()
    for b in range(batch):
        assert np.array_equal(C[b], go.gemm_i8(A[b], B if shared else B[b], D[b])), b


@pytest.mark.parametrize("m,n,k,rest_split", [
    (1100, 14336, 256, 1),    # 224 whole tiles + 56 partial: the split saves a round
    (2100, 8192, 1024, 1),    # 256 + 32: the remaining 52 rows on 64x64 tiles, K unsplit
    (4136, 4096, 1024, 2),    # 256 + 16: the remaining 40 rows on 64x64 tiles, K in 2 slices
])
def test_split_when_the_partial_row_adds_a_round(dev, m, n, k, rest_split):
    plan = hg.make_plan(m, n, k, has_d=True, d_max_abs=2**30, variant="mfma_256x256")
    top, rest = hg._mfma_parts(plan)
    assert top["m"] == m // 256 * 256 and rest["m"] == m % 256
    assert hg.mfma_k_split(rest) == rest_split
    ok, reason = hg.native_check(plan)
    assert ok and "%d rows on the persistent 256x256 kernel, %d on 128x128 tiles" % (
        top["m"], rest["m"]) in reason, reason
    say("edge tiles split", m, n, k)
    A, B, D = operands(m, n, k, m + n)
    At, Bt, Dt = to_dev(dev, A), to_dev(dev, B), to_dev(dev, D)
    C = hg.run(plan, At, Bt, Dt).cpu().numpy()
    C128 = hg.run(hg.make_plan(m, n, k, has_d=True, d_max_abs=2**30, variant="mfma_128x128"),
                  At, Bt, Dt).cpu().numpy()
    assert np.array_equal(C, C128)
    C2 = hg.run(plan, At, Bt, Dt, out=Dt).cpu().numpy()      # in place
    assert np.array_equal(C2, C)
    cut = m // 256 * 256
    for rows in (slice(0, 64), slice(cut - 64, cut + 16), slice(m - 40, m)):
        assert np.array_equal(C[rows], go.gemm_i8(A[rows], B, D[rows])), rows


def test_extremes_on_moved_back_tiles(dev):
    """K = 8192 with M and N both ragged: every product is the closed form."""
    m, n, k = 300, 528, 8192
    plan = hg.make_plan(m, n, k, variant="mfma_256x256")
    A = np.full((m, k), -128, np.int8)
    say("edge tiles extremes")
    assert np.all(hg.run(plan, to_dev(dev, A), to_dev(dev, np.full((k, n), -128, np.int8)))
                  .cpu().numpy() == 134217728)
    assert np.all(hg.run(plan, to_dev(dev, A), to_dev(dev, np.full((k, n), 127, np.int8)))
                  .cpu().numpy() == -133169152)


def test_large_ragged_problem(dev):
    """4000 x 4112 x 1024, both ragged, auto selection (256x256, 16 x 17
    tiles): the whole output passes the projection check and the rows
    around the moved-back tile row equal the oracle."""
    from veritac_amd.specializations.hip_gemm import verify
    m, n, k = 4000, 4112, 1024
    plan = hg.make_plan(m, n, k)
    assert plan["variant"] == "mfma_256x256" and hg._mfma_parts(plan) is None
    A, B, _ = operands(m, n, k, 99)
    At, Bt = to_dev(dev, A), to_dev(dev, B)
    say("edge tiles large")
    Ct = hg.run(plan, At, Bt)
    assert verify.exact_check(At, Bt, Ct)["passed"]
    C = Ct.cpu().numpy()
    for rows in (slice(3700, 3800), slice(m - 60, m)):
        assert np.array_equal(C[rows], go.gemm_i8_f64(A[rows], B)), rows


def test_split_with_unshared_batches(dev):
    """16 batches of 300 rows with their own B: 256 whole tiles and 256 partial
    ones, so every batch's whole 256-row tile runs in one persistent launch
    and every batch's last 44 rows in one batched launch of 128x128 tiles,
    out of place and in place."""
    batch, m, n, k = 16, 300, 4096, 256
    plan = hg.make_plan(m, n, k, batch=batch, has_d=True, d_max_abs=2**20,
                        variant="mfma_256x256")
    top, rest = hg._mfma_parts(plan)
    assert (top["m"], rest["m"], top["batch"], rest["batch"]) == (256, 44, batch, batch)
    rng = np.random.default_rng(31)
    A = rng.integers(-128, 128, (batch, m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (batch, k, n), dtype=np.int8)
    D = rng.integers(-2**20, 2**20, (batch, m, n), dtype=np.int32)
    At, Bt, Dt = to_dev(dev, A), to_dev(dev, B), to_dev(dev, D)
    say("edge tiles split, unshared batches")
    C = hg.run(plan, At, Bt, Dt).cpu().numpy()
    C2 = hg.run(plan, At, Bt, Dt, out=Dt).cpu().numpy()
    for b in range(batch):
        want = go.gemm_i8(A[b], B[b], D[b])
        assert np.array_equal(C[b], want), b
        assert np.array_equal(C2[b], want), b


@pytest.mark.parametrize("k", [2304, 320])
def test_padded_pitches_on_moved_back_tiles(dev, k):
    """A, B, C and D each with a padded pitch (lda = K + 64, ldb = N + 48,
    ldc = N + 4, ldd = N + 8) and M, N both ragged, on the 16x16x64 kernel
    (K = 2304) and the 32x32x32 one (K = 320): the DMA lane offsets and the
    masked stores follow the pitches, and the padding is never written."""
    m, n = 520, 784
    lda, ldb, ldc, ldd = k + 64, n + 48, n + 4, n + 8
    rng = np.random.default_rng(k + 5)
    Afull = rng.integers(-128, 128, (m, lda), dtype=np.int8)
    Bfull = rng.integers(-128, 128, (k, ldb), dtype=np.int8)
    Dfull = rng.integers(-2**20, 2**20, (m, ldd), dtype=np.int32)
    At, Bt, Dt = to_dev(dev, Afull), to_dev(dev, Bfull), to_dev(dev, Dfull)
    Cbuf = torch.full((m + 1, ldc), INT32_MIN, dtype=torch.int32, device=dev)
    say("edge tiles padded pitches", k)
    _lib.gemm_raw(At.data_ptr(), Bt.data_ptr(), Dt.data_ptr(), Cbuf.data_ptr(), m, n, k,
                  lda, ldb, ldd, ldc, variant="mfma_256x256")
    _lib.sync(None)
    got = Cbuf.cpu().numpy()
    want = go.gemm_i8(Afull[:, :k], Bfull[:, :n], Dfull[:, :n])
    assert np.array_equal(got[:m, :n], want)
    assert (got[:m, n:] == INT32_MIN).all() and (got[m:] == INT32_MIN).all()


def test_column_split_when_the_partial_column_adds_a_round(dev):
    """4096 x 4112 x 1024: 256 whole tiles plus 16 partial ones, so the whole
    4096 columns run on the persistent kernel and the last 16 on the 128x128
    variant (its 64x64 tiles on a grid this small) with K in 2 slices, out of
    place and in place."""
    m, n, k = 4096, 4112, 1024
    plan = hg.make_plan(m, n, k, has_d=True, d_max_abs=2**20, variant="mfma_256x256")
    top, rest = hg._mfma_parts(plan)
    assert (top["n"], rest["n"], hg.mfma_k_split(rest)) == (4096, 16, 2)
    A, B, D = operands(m, n, k, 17, d_bound=2**20)
    At, Bt, Dt = to_dev(dev, A), to_dev(dev, B), to_dev(dev, D)
    say("edge tiles column split")
    C = hg.run(plan, At, Bt, Dt).cpu().numpy()
    C128 = hg.run(hg.make_plan(m, n, k, has_d=True, d_max_abs=2**20, variant="mfma_128x128"),
                  At, Bt, Dt).cpu().numpy()
    assert np.array_equal(C, C128)
    C2 = hg.run(plan, At, Bt, Dt, out=Dt).cpu().numpy()
    assert np.array_equal(C2, C)
    assert np.array_equal(C[:, 4080:], go.gemm_i8(A, B[:, 4080:], D[:, 4080:]))
    for rows in (slice(0, 32), slice(m - 32, m)):
        assert np.array_equal(C[rows], go.gemm_i8(A[rows], B, D[rows])), rows

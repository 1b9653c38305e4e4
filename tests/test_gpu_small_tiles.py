"""The small tile levels of the mfma_128x128 variant against the oracle, through
the C ABI (needs a gfx950 GPU).

Row-major B on a small grid runs 64x128 tiles, or 64x64 tiles (one 32x32
accumulator block per wave, B slices of four 16-byte chunks per row) when
those also fit one workgroup per CU; each level takes its own K split. These
cases pin which level a shape takes (the host rule) and check every output:
whole tiles, ragged M and N (clamped loads, masked stores), K not a multiple
of 128 (the K-tail level), K of at most 128 (both slices in one round trip),
K split into slices summed by the reduction kernel, D (loaded before the k
loop on such grids), in place, D + A.B wrapping past int32 through the raw
C ABI, the int8 extremes, and batches.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import gemm_oracle as go
from veritac_amd import _lib
from veritac_amd.specializations.hip_gemm import backend as hg

pytestmark = pytest.mark.gpu


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


QUARTER, HALF = (64, 64), (64, 128)

# m, n, k, tile shape the plan runs, K slices
CASES = [
    (256, 256, 256, QUARTER, 1),      # config 2's shape: 16 whole tiles
    (64, 64, 64, QUARTER, 1),         # one tile, K of one slice
    (128, 128, 128, QUARTER, 1),      # K <= 128: both slices in one round trip
    (300, 208, 160, QUARTER, 1),      # ragged M and N, K % 128 != 0
    (192, 80, 320, QUARTER, 1),       # N: one whole and one partial 64-column tile
    (1024, 1024, 1024, QUARTER, 1),   # 256 tiles
    (512, 512, 2048, QUARTER, 4),     # 64 tiles, K in 4 slices of 512
    (96, 2048, 1024, QUARTER, 2),     # ragged M, K in 2 slices
    (256, 256, 8192, QUARTER, 16),    # 16 tiles, K in 16 slices
    (1024, 2048, 512, HALF, 1),       # 512 64x64 tiles: the 64x128 level
    (128, 4096, 4096, HALF, 4),       # 64x64 would leave K 4096 unsplit
]


@pytest.mark.parametrize("m,n,k,shape,ks", CASES)
def test_small_tiles_against_the_oracle(dev, m, n, k, shape, ks):
    plan = hg.make_plan(m, n, k, variant="mfma_128x128")
    assert (hg.mfma_tile_shape(plan), hg.mfma_k_split(plan)) == (shape, ks)
    _, _, _, native_ks, _ = _lib.gemm_check(m, n, k, k, n, n, n, variant="mfma_128x128")
    assert max(native_ks, 1) == ks
    rng = np.random.default_rng(m * 7 + n * 3 + k)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = rng.integers(-2**20, 2**20, (m, n), dtype=np.int32)
    At, Bt = to_dev(dev, A), to_dev(dev, B)
    say("small tiles", m, n, k, shape, ks)
    assert np.array_equal(hg.run(plan, At, Bt).cpu().numpy(), go.gemm_i8(A, B, None))
    plan_d = hg.make_plan(m, n, k, has_d=True, d_max_abs=2**20, variant="mfma_128x128")
    assert hg.mfma_tile_shape(plan_d) == shape
    # out of place, then in place (C = C + A.B)
    want = go.gemm_i8(A, B, D)
    assert np.array_equal(hg.run(plan_d, At, Bt, to_dev(dev, D)).cpu().numpy(), want)
    C = to_dev(dev, D)
    assert np.array_equal(hg.run(plan_d, At, Bt, C, out=C).cpu().numpy(), want)
    # past the int32 contract through the raw C ABI: D near both ends of
    # int32, so that D + A.B wraps (the mod 2^32 result the header promises)
    Dw = np.where(rng.integers(0, 2, (m, n)) == 1, 2**31 - 7, -2**31 + 7).astype(np.int32)
    Cw = to_dev(dev, Dw)
    _lib.gemm_raw(At.data_ptr(), Bt.data_ptr(), Cw.data_ptr(), Cw.data_ptr(), m, n, k, k, n, n, n,
                  1, 0, 0, 0, 0, "mfma_128x128", 0, None)
    _lib.sync(None)
    assert np.array_equal(Cw.cpu().numpy(), go.gemm_i8(A, B, Dw))


@pytest.mark.parametrize("m,n,k", [(256, 256, 256), (128, 192, 1024), (512, 512, 2048)])
def test_small_tiles_at_the_int8_extremes(dev, m, n, k):
    """All products at (-128)^2 and at -128 * 127: every slice's sum at the
    end of its range, through the K split where there is one."""
    plan = hg.make_plan(m, n, k, variant="mfma_128x128")
    assert hg.mfma_tile_shape(plan) == QUARTER
    for a, b in ((-128, -128), (-128, 127), (127, -128)):
        A = np.full((m, k), a, np.int8)
        B = np.full((k, n), b, np.int8)
        say("small tiles extremes", m, n, k, a, b)
        got = hg.run(plan, to_dev(dev, A), to_dev(dev, B)).cpu().numpy()
        assert np.array_equal(got, go.gemm_i8(A, B, None)), (a, b)


def test_small_tiles_on_batches(dev):
    """Unshared batches (each with its own B) of a 64x64-tile problem, and the
    same with D."""
    m, n, k, batch = 512, 512, 256, 4
    plan = hg.make_plan(m, n, k, batch=batch, variant="mfma_128x128")
    assert hg.mfma_tile_shape(plan) == QUARTER
    rng = np.random.default_rng(5)
    A = rng.integers(-128, 128, (batch, m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (batch, k, n), dtype=np.int8)
    D = rng.integers(-2**20, 2**20, (batch, m, n), dtype=np.int32)
    At, Bt, Dt = to_dev(dev, A), to_dev(dev, B), to_dev(dev, D)
    C = torch.empty((batch, m, n), dtype=torch.int32, device=dev)
    Cd = torch.empty_like(C)
    say("small tiles batches")
    _lib.gemm_raw(At.data_ptr(), Bt.data_ptr(), None, C.data_ptr(), m, n, k, k, n, n, n,
                  batch, m * k, k * n, 0, m * n, "mfma_128x128", 0, None)
    _lib.gemm_raw(At.data_ptr(), Bt.data_ptr(), Dt.data_ptr(), Cd.data_ptr(), m, n, k, k, n, n, n,
                  batch, m * k, k * n, m * n, m * n, "mfma_128x128", 0, None)
    _lib.sync(None)
    for i in range(batch):
        assert np.array_equal(C[i].cpu().numpy(), go.gemm_i8(A[i], B[i], None)), i
        assert np.array_equal(Cd[i].cpu().numpy(), go.gemm_i8(A[i], B[i], D[i])), i

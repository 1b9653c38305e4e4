"""gemm_dma16_kernel (full 256x256 tiles, K % 256 == 0, 8 x 8
v_mfma_i32_16x16x64_i8 accumulators per wave, C stored through an LDS strip as
16-byte row segments) against the oracle, through the C ABI (needs a gfx950
GPU). The 8192^3 headline shape and config 3 run on it and are checked by
their full-output hashes in test_gpu_config_hashes.py; these cases cover short
and long K, D in place, the int8 extremes, batches, packed B, and the C / D
alignment gate that sends other full-tile problems to the 32x32x32 kernel.
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


def run(dev, plan, A, B, D=None, in_place=False):
    At, Bt = to_dev(dev, A), to_dev(dev, B)
    if in_place:
        C = to_dev(dev, D)
        return hg.run(plan, At, Bt, C, out=C).cpu().numpy()
    Dt = to_dev(dev, D) if D is not None else None
    return hg.run(plan, At, Bt, Dt).cpu().numpy()


@pytest.mark.parametrize("m,n,k", [(256, 256, 256), (512, 256, 1024), (512, 512, 2048),
                                   (256, 512, 2304), (256, 256, 5120), (512, 256, 8192),
                                   (256, 768, 5376)])
def test_row_major_full_tiles(dev, m, n, k):
    say("dma16", m, n, k)
    rng = np.random.default_rng(m + n + k)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = rng.integers(-2**30, 2**30, (m, n), dtype=np.int32)
    plan = hg.make_plan(m, n, k, variant="mfma_256x256")
    assert np.array_equal(run(dev, plan, A, B), go.gemm_i8_f64(A, B))
    plan_d = hg.make_plan(m, n, k, has_d=True, d_max_abs=2**30, variant="mfma_256x256")
    want = go.gemm_i8(A, B, D)
    assert np.array_equal(run(dev, plan_d, A, B, D), want)
    assert np.array_equal(run(dev, plan_d, A, B, D, in_place=True), want)


def test_extremes_at_k8192(dev):
    m = n = 256
    k = 8192
    plan = hg.make_plan(m, n, k, variant="mfma_256x256")
    A = np.full((m, k), -128, np.int8)
    assert np.all(run(dev, plan, A, np.full((k, n), -128, np.int8)) == 134217728)
    assert np.all(run(dev, plan, A, np.full((k, n), 127, np.int8)) == -133169152)
    A = np.tile(np.array([-128, 127], np.int8), (m, k // 2))
    B = np.tile(np.array([[127], [-128]], np.int8), (k // 2, n))
    assert np.array_equal(run(dev, plan, A, B), go.gemm_i8_f64(A, B))
    # the largest partial sum a valid plan allows plus the largest product:
    # exactly 2^31 - 1
    dmax = 2**31 - 1 - 16384 * k
    plan_d = hg.make_plan(m, n, k, has_d=True, d_max_abs=dmax, variant="mfma_256x256")
    assert hg.validate_plan(plan_d)[0]
    A = np.full((m, k), -128, np.int8)
    C = run(dev, plan_d, A, np.full((k, n), -128, np.int8), np.full((m, n), dmax, np.int32))
    assert np.all(C == 2**31 - 1)


@pytest.mark.parametrize("shared", [True, False])
def test_batches(dev, shared):
    rng = np.random.default_rng(5 + shared)
    batch, m, n, k = 3, 256, 256, 5120
    A = rng.integers(-128, 128, (batch, m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n) if shared else (batch, k, n), dtype=np.int8)
    D = rng.integers(-1000, 1000, (batch, m, n), dtype=np.int32)
    plan = hg.make_plan(m, n, k, batch=batch, b_shared=shared, has_d=True, d_max_abs=1000,
                        variant="mfma_256x256")
    C = hg.run(plan, to_dev(dev, A), to_dev(dev, B), to_dev(dev, D)).cpu().numpy()
    for b in range(batch):
        assert np.array_equal(C[b], go.gemm_i8(A[b], B if shared else B[b], D[b])), b


def test_packed_dma_rows_equal_row_major_and_the_oracle(dev):
    """4096 x 2048 x 5120: 128 whole 256-row tiles on the packed DMA path; the
    full output equals the row-major kernel's and the 128x128 kernel's, and
    sampled rows equal the oracle."""
    m, n, k = 4096, 2048, 5120
    rng = np.random.default_rng(77)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    At, Bt = to_dev(dev, A), to_dev(dev, B)
    plan_p = hg.make_plan(m, n, k, variant=hg.PACKED_VARIANT)
    assert hg.packed_dma_rows(plan_p) == m
    Cp = hg.run(plan_p, At, hg.pack_b(Bt)).cpu().numpy()
    Cr = hg.run(hg.make_plan(m, n, k, variant="mfma_256x256"), At, Bt).cpu().numpy()
    C128 = hg.run(hg.make_plan(m, n, k, variant="mfma_128x128"), At, Bt).cpu().numpy()
    assert np.array_equal(Cp, Cr) and np.array_equal(Cr, C128)
    for rows in (slice(0, 256), slice(1792, 2048), slice(m - 256, m)):
        assert np.array_equal(Cr[rows], go.gemm_i8_f64(A[rows], B)), rows


@pytest.mark.parametrize("shared", [True, False])
def test_batches_without_d(dev, shared):
    """Without D the tile's last step stores six of its eight C strips (the
    rest after the loop); batches of unshared B are not folded, so tiles of
    every batch index run in one launch."""
    rng = np.random.default_rng(15 + shared)
    batch, m, n, k = 3, 512, 256, 1024
    A = rng.integers(-128, 128, (batch, m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n) if shared else (batch, k, n), dtype=np.int8)
    plan = hg.make_plan(m, n, k, batch=batch, b_shared=shared, variant="mfma_256x256")
    say("dma16 batches without D", shared)
    C = hg.run(plan, to_dev(dev, A), to_dev(dev, B)).cpu().numpy()
    for b in range(batch):
        assert np.array_equal(C[b], go.gemm_i8_f64(A[b], B if shared else B[b])), b


@pytest.mark.parametrize("k", [256, 4096])
def test_padded_ldc_without_d(dev, k):
    """ldc = N + 4: 16-byte rows with padding, early strips, padding untouched."""
    m, n = 256, 512
    ldc = n + 4
    rng = np.random.default_rng(k + 3)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    At, Bt = to_dev(dev, A), to_dev(dev, B)
    Cbuf = torch.full((m, ldc), INT32_MIN, dtype=torch.int32, device=dev)
    say("dma16 padded ldc without D", k)
    _lib.gemm_raw(At.data_ptr(), Bt.data_ptr(), None, Cbuf.data_ptr(), m, n, k, k, n, n, ldc,
                  variant="mfma_256x256")
    _lib.sync(None)
    C = Cbuf.cpu().numpy()
    assert np.array_equal(C[:, :n], go.gemm_i8_f64(A, B))
    assert (C[:, n:] == INT32_MIN).all()


@pytest.mark.parametrize("k", [2304, 4096])
def test_packed_dma_rows_with_d(dev, k):
    """Packed B with D on the 256x256 kernel: 4096 + 100 rows x 2048, the last
    tile row moved back to end at M (stores masked), out of place and in
    place."""
    m, n = 4096 + 100, 2048
    rng = np.random.default_rng(k)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = rng.integers(-2**30, 2**30, (m, n), dtype=np.int32)
    plan = hg.make_plan(m, n, k, has_d=True, d_max_abs=2**30, variant=hg.PACKED_VARIANT)
    assert hg.packed_dma_rows(plan) == m
    say("packed dma16 with D", m, n, k)
    At, Bp = to_dev(dev, A), hg.pack_b(to_dev(dev, B))
    Dt = to_dev(dev, D)
    C = hg.run(plan, At, Bp, Dt).cpu().numpy()
    C2 = hg.run(plan, At, Bp, Dt, out=Dt).cpu().numpy()
    for rows in (slice(0, 256), slice(2048, 2304), slice(3840, 4196)):
        want = go.gemm_i8(A[rows], B, D[rows])
        assert np.array_equal(C[rows], want), rows
        assert np.array_equal(C2[rows], want), rows
    assert np.array_equal(C, C2)


def test_k_not_a_multiple_of_256(dev):
    """K = 4160 and 320 (multiples of 64, not of 256) run on the 32x32x32
    kernel; both agree with the oracle."""
    rng = np.random.default_rng(9)
    for k in (4160, 320):
        A = rng.integers(-128, 128, (256, k), dtype=np.int8)
        B = rng.integers(-128, 128, (k, 256), dtype=np.int8)
        plan = hg.make_plan(256, 256, k, variant="mfma_256x256")
        assert np.array_equal(run(dev, plan, A, B), go.gemm_i8_f64(A, B)), k



@pytest.mark.parametrize("ldc,c_off,ldd,d_off", [
    (516, 0, 512, 0),      # 16-byte rows with padding: the 16x16x64 kernel
    (513, 0, 512, 0),      # ldc not a multiple of 4: 32x32x32
    (512, 1, 512, 0),      # C 4 bytes past a 16-byte boundary: 32x32x32
    (512, 0, 514, 0),      # ldd not a multiple of 4: 32x32x32
    (512, 0, 512, 3),      # D 12 bytes past a 16-byte boundary: 32x32x32
])
def test_c_and_d_alignment(dev, ldc, c_off, ldd, d_off):
    m, n, k = 256, 512, 1024
    say("dma16 alignment", ldc, c_off, ldd, d_off)
    rng = np.random.default_rng(ldc + 7 * c_off + ldd + 11 * d_off)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    Dfull = rng.integers(-2**20, 2**20, m * ldd + d_off, dtype=np.int32)
    D = Dfull[d_off:].reshape(m, ldd)
    At, Bt = to_dev(dev, A), to_dev(dev, B)
    Dt = to_dev(dev, Dfull)
    Cbuf = torch.full((m * ldc + c_off,), INT32_MIN, dtype=torch.int32, device=dev)
    _lib.gemm_raw(At.data_ptr(), Bt.data_ptr(), Dt.data_ptr() + 4 * d_off, Cbuf.data_ptr() + 4 * c_off,
                  m, n, k, k, n, ldd, ldc, variant="mfma_256x256")
    _lib.sync(None)
    got = Cbuf.cpu().numpy()
    C = got[c_off:].reshape(m, ldc)
    assert np.array_equal(C[:, :n], go.gemm_i8(A, B, D[:, :n]))
    assert (C[:, n:] == INT32_MIN).all() and (got[:c_off] == INT32_MIN).all()

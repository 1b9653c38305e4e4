"""Out-of-contract sums through the raw C ABI: every kernel family returns the
wrapped int32 sum, as include/vt_hip_gemm.h promises past the legality bound
k*16384 + |D| <= 2^31 - 1 (VeriTac/Gemmini/Word.lean:11, :31: a signed32
accumulator adds modulo 2^32).

Two ways out of range: an initial partial sum D within 2^12 of +-2^31 plus a
product that carries the sum across (the wrap happens where D is added), and
a K past 131071, where the products alone leave int32 (the wrap happens in
the MFMA accumulators, or in the K-split reduction). Each case reaches the
kernel named beside it (variant and K split checked on the host by
vt_gemm_check) and compares with the oracle's exact sum wrapped to int32
(needs a gfx950 GPU)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import gemm_oracle as go
from veritac_amd import _lib

pytestmark = pytest.mark.gpu

INT32_MIN, INT32_MAX = -2**31, 2**31 - 1
K_LONG = 139264          # > 131071 = (2^31 - 1) // 16384, a multiple of 256


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    assert _lib.load_library().vt_device_count() >= 1, "GPU visible but not gfx950"
    return torch.device("cuda", 0)


def near_limits(rng, shape):
    """int32 D within 2^12 of INT32_MAX or INT32_MIN, half each."""
    off = rng.integers(0, 1 << 12, shape, dtype=np.int64)
    top = rng.integers(0, 2, shape).astype(bool)
    return np.where(top, INT32_MAX - off, INT32_MIN + off).astype(np.int32)


def run_raw(dev, A, B, D, variant, k_split, want_split, in_place=False):
    m, k = A.shape
    n = B.shape[1]
    st = _lib.gemm_check(m, n, k, k, n, n, n, has_d=True, variant=variant, k_split=k_split)
    assert st[0] == _lib.VT_OK and st[3] == want_split, st
    At, Bt = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
    Dt = torch.from_numpy(D).to(dev)
    Ct = Dt if in_place else torch.empty((m, n), dtype=torch.int32, device=dev)
    _lib.gemm_raw(At.data_ptr(), Bt.data_ptr(), Dt.data_ptr(), Ct.data_ptr(), m, n, k, k, n, n, n,
                  variant=variant, k_split=k_split)
    _lib.sync(None)
    return Ct.cpu().numpy()


# (variant, k_split asked, M, N, K, K split that runs): the kernel each reaches
D_CASES = [
    ("generic", 0, 64, 64, 256, 0),             # generic_kernel (VALU)
    ("mfma_128x128", 0, 256, 256, 512, 0),      # gemm_mfma_kernel<128,128>
    ("mfma_256x128", 0, 256, 256, 512, 0),      # gemm_mfma_kernel<256,128>
    ("mfma_256x256", 0, 2304, 2048, 1024, 0),   # gemm_dma16_kernel (72 tiles, no split)
    ("mfma_256x256", 0, 2100, 2064, 1024, 0),   # gemm_dma16_kernel, moved-back edge tiles
    ("mfma_256x256", 0, 2304, 2048, 320, 0),    # gemm_dma_kernel (32x32x32; K % 256 != 0)
    ("mfma_256x256", 0, 512, 512, 1024, 2),     # K split into partials + skinny_reduce_kernel
    ("skinny", 1, 16, 2048, 4096, 1),           # skinny_kernel, whole K, D in its epilogue
    ("skinny", 4, 16, 2048, 4096, 4),           # skinny_kernel + skinny_reduce_kernel
    ("skinny", 0, 1, 1024, 2048, 16),           # M = 1 decode
    ("padded", 0, 40, 72, 100, 0),              # pad copies + vector kernel + unpad
]


@pytest.mark.parametrize("variant,k_split,m,n,k,split", D_CASES)
def test_partial_sum_near_int32_limits_wraps(dev, variant, k_split, m, n, k, split):
    print("wrap D", variant, k_split, m, n, k, flush=True)
    rng = np.random.default_rng(m * 7 + n + k)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = near_limits(rng, (m, n))
    want = go.gemm_i8(A, B, D)
    exact = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.int64) + D
    crossed = (exact > INT32_MAX) | (exact < INT32_MIN)
    assert crossed.mean() > 0.25       # the case does leave the int32 range
    assert np.array_equal(want, (exact + 2**31) % 2**32 - 2**31)   # the oracle wraps
    assert np.array_equal(run_raw(dev, A, B, D, variant, k_split, split), want)
    if variant == "mfma_256x256" and split == 0 and k % 256 == 0:
        assert np.array_equal(run_raw(dev, A, B, D.copy(), variant, k_split, split, in_place=True),
                              want)


@pytest.mark.parametrize("variant,m,n,split", [
    ("generic", 16, 16, 0),                 # VALU sum wraps
    ("skinny", 16, 256, 64),                # partials in range; the reduction wraps
    ("mfma_128x128", 256, 256, 16),         # K split; the reduction wraps
    ("mfma_256x256", 2304, 4096, 0)])       # gemm_dma16_kernel (144 tiles, K unsplit): the
                                            # MFMA accumulators wrap
def test_k_past_the_legality_bound_wraps(dev, variant, m, n, split):
    """All -128 operands over K = 139264 give 16384 * K = 2281701376 per cell
    before D, which wraps to -2013265920; then mixed signs, checked against
    the oracle on the first and last 256 x 256 output tiles."""
    k = K_LONG
    print("wrap K", variant, m, n, k, flush=True)
    rng = np.random.default_rng(k + m)
    A = np.full((m, k), -128, np.int8)
    B = np.full((k, n), -128, np.int8)
    D = rng.integers(-1000, 1000, (m, n), dtype=np.int32)
    want = ((16384 * k + D.astype(np.int64)) & 0xFFFFFFFF).astype(np.uint32).view(np.int32)
    t = min(m, 256), min(n, 256)
    assert np.array_equal(want[:t[0], :t[1]], go.gemm_i8_f64(A[:t[0]], B[:, :t[1]], D[:t[0], :t[1]]))
    assert np.array_equal(run_raw(dev, A, B, D, variant, 0, split), want)
    # the last 4096 products random: 16384 * 135168 plus a tail of either sign
    A[:, k - 4096:] = rng.integers(-128, 128, (m, 4096), dtype=np.int8)
    B[k - 4096:] = rng.integers(-128, 128, (4096, n), dtype=np.int8)
    C = run_raw(dev, A, B, D, variant, 0, split)
    for rows, cols in ((slice(0, t[0]), slice(0, t[1])), (slice(m - t[0], m), slice(n - t[1], n))):
        assert np.array_equal(C[rows, cols], go.gemm_i8_f64(A[rows], B[:, cols], D[rows, cols]))


def test_packed_paths_wrap(dev):
    """vt_gemm_i8_packed: the decode kernel at M = 16 and packed 128x128 tiles
    at M = 512 with D near the int32 limits, and the decode kernel over
    K = 139264 in one pass, where its MFMA accumulators wrap."""
    rng = np.random.default_rng(99)
    for m, n, k in ((16, 2048, 4096), (512, 2048, 4096), (16, 256, K_LONG)):
        print("wrap packed", m, n, k, flush=True)
        A = rng.integers(-128, 128, (m, k), dtype=np.int8)
        B = rng.integers(-128, 128, (k, n), dtype=np.int8)
        if k == K_LONG:      # 16384 * 135168 plus a random tail: past 2^31
            A[:, : k - 4096] = -128
            B[: k - 4096] = -128
            D = rng.integers(-1000, 1000, (m, n), dtype=np.int32)
        else:
            D = near_limits(rng, (m, n))
        Bt = torch.from_numpy(B).to(dev)
        Bp = torch.empty(_lib.packed_b_size(k, n), dtype=torch.int8, device=dev)
        _lib.pack_b_raw(Bt.data_ptr(), Bp.data_ptr(), k, n, n)
        At, Dt = torch.from_numpy(A).to(dev), torch.from_numpy(D).to(dev)
        Ct = torch.empty((m, n), dtype=torch.int32, device=dev)
        # one pass over K (k_split 1): at N = 256 the default would split K
        _lib.gemm_packed_raw(At.data_ptr(), Bp.data_ptr(), Dt.data_ptr(), Ct.data_ptr(), m, n, k,
                             k, n, n, k_split=1)
        _lib.sync(None)
        want = go.gemm_i8_f64(A, B, D)
        if k == K_LONG:
            assert (want > 0).mean() < 0.5      # most sums wrapped to negative values
        assert np.array_equal(Ct.cpu().numpy(), want), (m, n, k)

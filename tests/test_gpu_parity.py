"""Bit-exact parity of the HIP kernels with the CPU oracle (needs a gfx950 GPU).

Every call goes through the C ABI (veritac_amd._lib -> libvt_hip_gemm.so).
Outputs are poisoned with INT32_MIN before each launch (the reference's
emitted-C harness does the same, backend.py:756-760) so unwritten cells show.
Small and medium shapes are compared element by element with the oracle;
the full-size benchmark shapes are checked with exact int64/float64
properties (row and column checksums, Freivalds products, full sampled rows
and columns) that any wrong element fails with overwhelming probability.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from conftest import decode_cout
from oracle import cref
from oracle import gemm_oracle as go
from veritac_amd import _lib
from veritac_amd.specializations.hip_gemm import backend as hg
from veritac_amd.specializations.hip_gemm import inputs

pytestmark = pytest.mark.gpu

INT32_MIN = -2**31
VEC_VARIANTS = ("mfma_256x256", "mfma_256x128", "mfma_128x128")


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    lib = _lib.load_library()
    assert lib.vt_device_count() >= 1, "GPU visible but not gfx950"
    return torch.device("cuda", 0)


def say(*args):
    print(*args, flush=True)


def gpu_gemm(dev, A, B, D=None, variant="auto", k_split=0, batch_shared=False):
    """Run C = D + A.B through the C ABI with explicit pointers and strides."""
    At = torch.from_numpy(np.ascontiguousarray(A)).to(dev)
    Bt = torch.from_numpy(np.ascontiguousarray(B)).to(dev)
    Dt = torch.from_numpy(np.ascontiguousarray(D)).to(dev) if D is not None else None
    batched = At.dim() == 3
    b = At.shape[0] if batched else 1
    M, K = At.shape[-2:]
    N = Bt.shape[-1]
    C = torch.full((b, M, N) if batched else (M, N), INT32_MIN, dtype=torch.int32, device=dev)
    _lib.gemm_raw(At.data_ptr(), Bt.data_ptr(), Dt.data_ptr() if Dt is not None else None,
                  C.data_ptr(), M, N, K, K, N, N, N, b,
                  M * K if batched else 0, (K * N if Bt.dim() == 3 else 0),
                  M * N if (batched and Dt is not None) else 0, M * N if batched else 0,
                  variant, k_split, None)
    _lib.sync(None)
    return C.cpu().numpy()


# ---------------------------------------------------------------------------
# Golden vectors (recorded Spike outputs) through every kernel
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("variant", ["auto", "mfma_128x128", "mfma_256x256", "mfma_256x128",
                                     "skinny", "generic"])
def test_spike_golden_vectors(dev, golden, variant):
    for run in golden["runs"]:
        m, n, k = run["plan"]["m"], run["plan"]["n"], run["plan"]["k"]
        if variant == "skinny" and m > 64:
            continue
        for mode in golden["modes"]:
            say("golden", run["name"], mode, variant)
            A, B = inputs.spike_inputs(mode, m, n, k)
            want = np.array(decode_cout(run["cout"][mode]), np.int32).reshape(m, n)
            assert np.array_equal(gpu_gemm(dev, A, B, variant=variant), want), (run["name"], mode)


# ---------------------------------------------------------------------------
# The benchmark configurations
# ---------------------------------------------------------------------------

def test_config1_64cube(dev):
    for seed in (0, 1, 2):
        c = inputs.config_inputs(1, seed=seed)
        say("config1 seed", seed)
        for variant in ("auto", "mfma_128x128", "generic"):
            assert np.array_equal(gpu_gemm(dev, c["A"], c["B"], variant=variant),
                                  go.gemm_i8(c["A"], c["B"])), (seed, variant)


def test_config2_partial_sum_256(dev):
    for seed in (0, 5):
        c = inputs.config_inputs(2, seed=seed)
        want = go.gemm_i8_ktiled(c["A"], c["B"], c["D"], k_tile=16)
        assert np.array_equal(want, go.gemm_i8_int64(c["A"], c["B"], c["D"]))
        for variant in ("auto",) + VEC_VARIANTS + ("generic",):
            say("config2 seed", seed, variant)
            assert np.array_equal(gpu_gemm(dev, c["A"], c["B"], c["D"], variant=variant), want)


def test_config2_mutation_is_detected(dev):
    """A planted mistake in the oracle (D dropped) must not match the GPU."""
    c = inputs.config_inputs(2, seed=3)
    got = gpu_gemm(dev, c["A"], c["B"], c["D"])
    assert np.array_equal(got, go.gemm_i8(c["A"], c["B"], c["D"]))
    assert not np.array_equal(got, go.gemm_i8(c["A"], c["B"]))          # D dropped
    bad_tiles = go.gemm_i8_int64(c["A"][:, 16:], c["B"][16:, :], c["D"])  # first K tile lost
    assert not np.array_equal(got, bad_tiles)


def test_config3_batched_b_reuse(dev):
    c = inputs.config_inputs(3, seed=0)
    A, B = c["A"], c["B"]
    want = go.gemm_i8_f64(A, B)
    for variant in ("auto", "mfma_256x256", "mfma_128x128"):
        say("config3", variant)
        got = gpu_gemm(dev, A, B, variant=variant)
        assert np.array_equal(got, want), variant


@pytest.mark.parametrize("m", [1, 16])
def test_config4_decode(dev, m):
    c = inputs.config_inputs(4, seed=m, m=m)
    want = go.gemm_i8_f64(c["A"], c["B"])
    for ks in (0, 1, 2, 4, 7):
        say("config4 m", m, "k_split", ks)
        got = gpu_gemm(dev, c["A"], c["B"], variant="skinny", k_split=ks)
        assert np.array_equal(got, want), ks
    assert np.array_equal(gpu_gemm(dev, c["A"], c["B"]), want)


def _exact_properties(A, B, C, rng, samples=48):
    """Exact checks of C == A.B for large shapes (no int32 wrap in contract)."""
    Af = A.astype(np.float64)
    Bf = B.astype(np.float64)
    Cf = C.astype(np.float64)
    # row and column checksums (checksum of checksums)
    assert np.array_equal(Cf.sum(axis=1), Af @ Bf.sum(axis=1))
    assert np.array_equal(Cf.sum(axis=0), Af.sum(axis=0) @ Bf)
    # Freivalds with random small-integer vectors (exact in float64)
    for _ in range(2):
        x = rng.integers(-3, 4, size=B.shape[1]).astype(np.float64)
        assert np.array_equal(Cf @ x, Af @ (Bf @ x))
    # full sampled rows and columns against the exact product
    rows = rng.choice(A.shape[0], size=samples, replace=False)
    cols = rng.choice(B.shape[1], size=samples, replace=False)
    assert np.array_equal(C[rows], go.gemm_i8_f64(A[rows], B))
    assert np.array_equal(C[:, cols], go.gemm_i8_f64(A, B[:, cols]))


def test_config5_8192_adversarial(dev):
    c = inputs.config_inputs(5, seed=0)
    A, B = c["A"], c["B"]
    assert np.count_nonzero((A == -128) | (A == 127)) > A.size * 0.45
    say("config5 auto")
    got = gpu_gemm(dev, A, B)
    assert (got != INT32_MIN).all()
    _exact_properties(A, B, got, np.random.default_rng(0))


def test_extremes_at_the_overflow_edge(dev):
    # all -128: every output is K*16384; at K=8192 that is 134217728 (< 2^31)
    for (m, n, k) in ((256, 256, 8192), (16, 256, 8192), (300, 144, 4096)):
        A = np.full((m, k), -128, np.int8)
        B = np.full((k, n), -128, np.int8)
        for variant in ("auto", "generic"):
            say("extremes", m, n, k, variant)
            got = gpu_gemm(dev, A, B, variant=variant)
            assert (got == k * 16384).all()
        A2 = np.where(np.arange(m * k).reshape(m, k) % 2 == 0, -128, 127).astype(np.int8)
        B2 = np.where(np.arange(k * n).reshape(k, n) % 3 == 0, 127, -128).astype(np.int8)
        assert np.array_equal(gpu_gemm(dev, A2, B2), go.gemm_i8_f64(A2, B2))


# ---------------------------------------------------------------------------
# Edge shapes, tails, strides, in-place and repeated calls
# ---------------------------------------------------------------------------

EDGE_SHAPES = [(1, 16, 16), (17, 48, 80), (129, 144, 64), (300, 272, 208), (255, 256, 320),
               (257, 128, 1040), (33, 16, 4112), (512, 512, 64), (16, 14352, 4160),
               (3, 2064, 1024), (640, 384, 48)]


@pytest.mark.parametrize("shape", EDGE_SHAPES)
def test_edge_shapes_all_variants(dev, shape):
    m, n, k = shape
    rng = np.random.default_rng(m * 7 + n * 3 + k)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = rng.integers(-(1 << 20), (1 << 20) + 1, (m, n), dtype=np.int32)
    want = go.gemm_i8(A, B)
    want_d = go.gemm_i8(A, B, D)
    variants = ["auto", "generic"] + list(VEC_VARIANTS) + (["skinny"] if m <= 64 else [])
    for variant in variants:
        say("edge", shape, variant)
        assert np.array_equal(gpu_gemm(dev, A, B, variant=variant), want), variant
        assert np.array_equal(gpu_gemm(dev, A, B, D, variant=variant), want_d), variant


def test_unaligned_shapes_use_generic(dev):
    rng = np.random.default_rng(11)
    for (m, n, k) in ((5, 7, 9), (33, 20, 50), (2, 3, 1)):
        A = rng.integers(-128, 128, (m, k), dtype=np.int8)
        B = rng.integers(-128, 128, (k, n), dtype=np.int8)
        say("unaligned", m, n, k)
        assert np.array_equal(gpu_gemm(dev, A, B), go.gemm_i8(A, B))
        with pytest.raises(_lib.HipGemmError):
            gpu_gemm(dev, A, B, variant="mfma_128x128")


def test_strided_operands_and_inplace(dev):
    rng = np.random.default_rng(5)
    m, n, k = 200, 160, 96
    lda, ldb, ldc = k + 32, n + 16, n + 48
    Abuf = torch.from_numpy(rng.integers(-128, 128, (m, lda), dtype=np.int8)).to(dev)
    Bbuf = torch.from_numpy(rng.integers(-128, 128, (k, ldb), dtype=np.int8)).to(dev)
    D0 = rng.integers(-1000, 1000, (m, ldc), dtype=np.int32)
    A = Abuf[:, :k].cpu().numpy()
    B = Bbuf[:, :n].cpu().numpy()
    want = go.gemm_i8(A, B, D0[:, :n])
    for variant in ("auto", "mfma_128x128", "mfma_256x128", "generic"):
        say("strided in-place", variant)
        Cbuf = torch.from_numpy(D0.copy()).to(dev)
        # in place: D and C are the same buffer
        _lib.gemm_raw(Abuf.data_ptr(), Bbuf.data_ptr(), Cbuf.data_ptr(), Cbuf.data_ptr(),
                      m, n, k, lda, ldb, ldc, ldc, variant=variant)
        _lib.sync(None)
        got = Cbuf.cpu().numpy()
        assert np.array_equal(got[:, :n], want), variant
        assert np.array_equal(got[:, n:], D0[:, n:]), variant   # padding untouched


def test_batched_unshared_and_shared(dev):
    rng = np.random.default_rng(9)
    b, m, n, k = 5, 48, 144, 80
    A = rng.integers(-128, 128, (b, m, k), dtype=np.int8)
    Bs = rng.integers(-128, 128, (b, k, n), dtype=np.int8)
    D = rng.integers(-50, 50, (b, m, n), dtype=np.int32)
    for variant in ("auto", "mfma_128x128", "generic"):
        say("batched", variant)
        assert np.array_equal(gpu_gemm(dev, A, Bs, D, variant=variant), go.gemm_i8(A, Bs, D))
        assert np.array_equal(gpu_gemm(dev, A, Bs[0], variant=variant), go.gemm_i8(A, Bs[0]))
    A16 = A[:, :16, :]
    assert np.array_equal(gpu_gemm(dev, np.ascontiguousarray(A16), Bs, variant="skinny", k_split=2),
                          go.gemm_i8(A16, Bs))


@pytest.mark.parametrize("m", [17, 24, 31, 32, 33, 48, 63, 64])
@pytest.mark.parametrize("k_split", [0, 1, 3])
def test_skinny_row_blocks(dev, m, k_split):
    """17..64 rows run as 2 or 4 row blocks of 16 over the same B stream:
    rows past M are zero in the A slice and never stored; D added in place."""
    rng = np.random.default_rng(m * 10 + k_split)
    n, k = 1040, 4160
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = rng.integers(-(1 << 20), (1 << 20) + 1, (m, n), dtype=np.int32)
    say("skinny row blocks", m, "k_split", k_split)
    assert np.array_equal(gpu_gemm(dev, A, B, variant="skinny", k_split=k_split), go.gemm_i8(A, B))
    At, Bt = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
    C = torch.from_numpy(D).to(dev)          # C = D + A.B in place
    _lib.gemm_raw(At.data_ptr(), Bt.data_ptr(), C.data_ptr(), C.data_ptr(), m, n, k, k, n, n, n,
                  1, 0, 0, 0, 0, "skinny", k_split, None)
    _lib.sync(None)
    assert np.array_equal(C.cpu().numpy(), go.gemm_i8(A, B, D))


def test_skinny_row_blocks_extremes(dev):
    m, k, n = 64, 8192, 256
    A = np.full((m, k), -128, np.int8)
    B = np.full((k, n), -128, np.int8)
    assert np.all(gpu_gemm(dev, A, B, variant="skinny") == 134217728)
    A = np.tile(np.array([-128, 127], np.int8), (m, k // 2))
    B = np.tile(np.array([[127], [-128]], np.int8), (k // 2, n))
    assert np.array_equal(gpu_gemm(dev, A, B, variant="skinny", k_split=5), go.gemm_i8_f64(A, B))


def test_skinny_repeated_calls_reset_counters(dev):
    rng = np.random.default_rng(21)
    for it in range(4):
        m = (1, 16, 7, 16)[it]
        A = rng.integers(-127, 128, (m, 2048), dtype=np.int8)
        B = rng.integers(-128, 128, (2048, 4096), dtype=np.int8)
        say("skinny repeat", it, m)
        assert np.array_equal(gpu_gemm(dev, A, B, variant="skinny", k_split=4), go.gemm_i8(A, B))


def test_backend_run_on_side_stream(dev):
    rng = np.random.default_rng(2)
    A = torch.from_numpy(rng.integers(-128, 128, (384, 256), dtype=np.int8)).to(dev)
    B = torch.from_numpy(rng.integers(-128, 128, (256, 512), dtype=np.int8)).to(dev)
    plan = hg.make_plan(384, 512, 256)
    s = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(s):
        C = hg.run(plan, A, B)
    s.synchronize()
    want = go.gemm_i8(A.cpu().numpy(), B.cpu().numpy())
    assert np.array_equal(C.cpu().numpy(), want)
    # a raw stream handle while torch's current stream stays the default one:
    # outputs allocated here are recorded as used on it
    s.wait_stream(torch.cuda.current_stream(dev))
    C2 = hg.run(plan, A, B, stream=s.cuda_stream)
    W = B[:, :256].contiguous()
    Bp = hg.pack_b(W, stream=s.cuda_stream)
    x = A[:16].contiguous()
    C3 = hg.run(hg.make_plan(16, 256, 256, variant="skinny_packed"), x, Bp, stream=s.cuda_stream)
    s.synchronize()
    assert np.array_equal(C2.cpu().numpy(), want)
    assert np.array_equal(C3.cpu().numpy(), want[:16, :256])
    flat = hg.run_flat(hg.make_plan(16, 16, 16), [1] * 256, [-2] * 256)
    assert flat == [-32] * 256


def test_cpu_reference_agrees_on_gpu_box(dev):
    """The C oracle built for this host agrees with the GPU on a mid-size case."""
    rng = np.random.default_rng(4)
    A = rng.integers(-128, 128, (96, 512), dtype=np.int8)
    B = rng.integers(-128, 128, (512, 320), dtype=np.int8)
    assert np.array_equal(gpu_gemm(dev, A, B), cref.gemm_i8(A, B, order="ikj"))


FULL_TILE_SHAPES = [(256, 256, 64), (256, 512, 192), (512, 256, 1088), (768, 512, 4096),
                    (256, 256, 128)]


@pytest.mark.parametrize("shape", FULL_TILE_SHAPES)
def test_full_tile_dma_path(dev, shape):
    """Shapes made of whole 256x256 tiles take the direct-to-LDS kernel."""
    m, n, k = shape
    rng = np.random.default_rng(m + 3 * n + 7 * k)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = rng.integers(-(1 << 20), (1 << 20) + 1, (m, n), dtype=np.int32)
    say("full tile", shape)
    assert np.array_equal(gpu_gemm(dev, A, B, variant="mfma_256x256"), go.gemm_i8(A, B))
    assert np.array_equal(gpu_gemm(dev, A, B, D, variant="mfma_256x256"), go.gemm_i8(A, B, D))
    # batched, one B per batch (no stacked-M fold), with D
    A3 = rng.integers(-128, 128, (3, m, k), dtype=np.int8)
    B3 = rng.integers(-128, 128, (3, k, n), dtype=np.int8)
    D3 = rng.integers(-99, 99, (3, m, n), dtype=np.int32)
    assert np.array_equal(gpu_gemm(dev, A3, B3, D3, variant="mfma_256x256"), go.gemm_i8(A3, B3, D3))


# Persistent-kernel shapes where workgroups walk several tiles, some one more
# than others (529 and 600 tiles over 256 workgroups), k loops of 2 and of an
# odd 3 slices (the slice stream crosses tile boundaries every few steps),
# batches walked by one grid, repeated into poisoned outputs.
MULTI_TILE_SHAPES = [(5120, 7680, 512, 1), (5888, 5888, 128, 1), (4096, 8192, 192, 1),
                     (2048, 2048, 320, 8)]


@pytest.mark.parametrize("shape", MULTI_TILE_SHAPES)
def test_persistent_multi_tile_walks(dev, shape):
    """Every workgroup of the persistent kernel walks two or more tiles, with
    and without D; with D also in place (C is D's buffer)."""
    m, n, k, batch = shape
    rng = np.random.default_rng(m + n + k + batch)
    A = rng.integers(-128, 128, (batch, m, k) if batch > 1 else (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (batch, k, n) if batch > 1 else (k, n), dtype=np.int8)
    D = rng.integers(-(1 << 20), (1 << 20) + 1, (batch, m, n) if batch > 1 else (m, n),
                     dtype=np.int32)
    tiles = batch * (m // 256) * (n // 256)
    assert tiles >= 512, "shape must give every workgroup at least two tiles"
    say("multi-tile", shape, "tiles", tiles)
    want = go.gemm_i8(A, B)
    for _ in range(3):
        assert np.array_equal(gpu_gemm(dev, A, B, variant="mfma_256x256"), want), shape
    want_d = (want.astype(np.int64) + D).astype(np.int32)
    assert np.array_equal(gpu_gemm(dev, A, B, D, variant="mfma_256x256"), want_d), shape
    if batch == 1:
        At, Bt = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
        Ct = torch.from_numpy(D).to(dev)
        plan = hg.make_plan(m, n, k, has_d=True, d_max_abs=1 << 20, variant="mfma_256x256")
        hg.run(plan, At, Bt, Ct, out=Ct)
        assert np.array_equal(Ct.cpu().numpy(), want_d), shape


# K of at most 128: one pair of k steps, the SHORT instantiation (both slices
# fetched in one round trip), on edge and whole tiles, with and without D
SHORT_K_SHAPES = [(64, 64, 64), (128, 128, 128), (200, 304, 16), (256, 256, 80),
                  (384, 512, 128), (130, 144, 48), (512, 256, 64)]


@pytest.mark.parametrize("variant", ["mfma_128x128", "mfma_256x128", "mfma_256x256"])
@pytest.mark.parametrize("shape", SHORT_K_SHAPES)
def test_short_k_path(dev, shape, variant):
    m, n, k = shape
    rng = np.random.default_rng(m * 7 + n * 3 + k)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = rng.integers(-(1 << 20), (1 << 20) + 1, (m, n), dtype=np.int32)
    say("short k", shape, variant)
    assert np.array_equal(gpu_gemm(dev, A, B, variant=variant), go.gemm_i8(A, B))
    assert np.array_equal(gpu_gemm(dev, A, B, D, variant=variant), go.gemm_i8(A, B, D))


def test_full_tile_repeated_launches_are_stable(dev):
    """Many back-to-back launches of the pipelined kernels give identical,
    exact results (a stage published too early would show as a mismatch)."""
    rng = np.random.default_rng(77)
    m = n = 1024
    k = 2048
    A = torch.from_numpy(rng.integers(-128, 128, (m, k), dtype=np.int8)).to(dev)
    B = torch.from_numpy(rng.integers(-128, 128, (k, n), dtype=np.int8)).to(dev)
    want = go.gemm_i8(A.cpu().numpy(), B.cpu().numpy())
    for variant in ("mfma_256x256", "mfma_256x128", "mfma_128x128"):
        outs = [torch.full((m, n), INT32_MIN, dtype=torch.int32, device=dev) for _ in range(20)]
        for C in outs:
            _lib.gemm_raw(A.data_ptr(), B.data_ptr(), None, C.data_ptr(), m, n, k, k, n, n, n,
                          variant=variant)
        _lib.sync(None)
        say("repeat", variant)
        for C in outs:
            assert np.array_equal(C.cpu().numpy(), want), variant


# (m, n, k, batch, with_d): decode-sized skinny problems -- a single k slice
# (K = 64), K not a multiple of the slice pipeline (4160), M of 1 / 3 / 7 / 15,
# an initial partial sum and two batches.
DECODE_SHAPES = [(16, 8192, 4096, 1, False), (1, 8192, 64, 1, True), (3, 8192, 128, 1, False),
                 (15, 8192, 4160, 1, True), (16, 4096, 512, 2, True), (7, 14336, 1024, 1, False)]


@pytest.mark.parametrize("shape", DECODE_SHAPES)
def test_decode_kernel_shapes(dev, shape):
    m, n, k, b, with_d = shape
    say("decode shape", shape)
    assert _lib.select_variant(m, n, k, b, k, n, True)[0] == "skinny"
    rng = np.random.default_rng(m * 7 + k)
    A = rng.integers(-128, 128, (b, m, k) if b > 1 else (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (b, k, n) if b > 1 else (k, n), dtype=np.int8)
    D = rng.integers(-2**20, 2**20, A.shape[:-1] + (n,), dtype=np.int32) if with_d else None
    want = go.gemm_i8_f64(A, B, D)
    assert np.array_equal(gpu_gemm(dev, A, B, D), want)
    for ks in (1, 3):
        assert np.array_equal(gpu_gemm(dev, A, B, D, variant="skinny", k_split=ks), want)


def test_decode_kernel_padded_strides(dev):
    m, n, k = 16, 8192, 2048
    lda, ldb, ldc = k + 80, n + 128, n + 48
    rng = np.random.default_rng(5)
    Ap = rng.integers(-128, 128, (m, lda), dtype=np.int8)
    Bp = rng.integers(-128, 128, (k, ldb), dtype=np.int8)
    want = go.gemm_i8_f64(Ap[:, :k], Bp[:, :n])
    At = torch.from_numpy(Ap).to(dev)
    Bt = torch.from_numpy(Bp).to(dev)
    Ct = torch.full((m, ldc), INT32_MIN, dtype=torch.int32, device=dev)
    _lib.gemm_raw(At.data_ptr(), Bt.data_ptr(), None, Ct.data_ptr(), m, n, k, lda, ldb, n, ldc,
                  variant="skinny", k_split=0)
    _lib.sync(None)
    got = Ct.cpu().numpy()
    assert np.array_equal(got[:, :n], want)
    assert (got[:, n:] == INT32_MIN).all()


# ---------------------------------------------------------------------------
# The padded variant: any shape through the vector kernels
# ---------------------------------------------------------------------------

PADDED_SHAPES = [(1000, 1000, 1000, 1), (1001, 999, 1003, 1), (16, 14335, 4095, 1),
                 (1, 4097, 4095, 1), (300, 500, 1000, 3), (5, 7, 9, 1),
                 # N % 16 == 0: the product writes C and adds D itself
                 (500, 2000, 1500, 1), (200, 512, 777, 3), (7, 4096, 1001, 1),
                 # K % 16 == 0: A is read in place, only B is copied
                 (300, 1001, 1024, 1), (16, 14335, 4096, 1), (100, 333, 512, 2),
                 # aligned: nothing is copied
                 (256, 256, 256, 1), (64, 512, 512, 2)]


@pytest.mark.parametrize("shape", PADDED_SHAPES)
def test_padded_variant(dev, shape):
    """K and N not multiples of 16: zero-padded copies of the operands that
    need them through the MFMA or skinny kernel, then C (plus D, also in
    place) copied out or, when N % 16 == 0, written by the product; compared
    with the C oracle and with the VALU kernel."""
    m, n, k, batch = shape
    rng = np.random.default_rng(m + n + k + batch)
    A = rng.integers(-128, 128, (batch, m, k) if batch > 1 else (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)        # shared by every batch
    D = rng.integers(-(1 << 20), (1 << 20) + 1, (batch, m, n) if batch > 1 else (m, n),
                     dtype=np.int32)
    say("padded", shape)
    if batch == 1:
        want = cref.gemm_i8(A, B, order="ikj")
    else:
        want = np.stack([cref.gemm_i8(A[b], B, order="ikj") for b in range(batch)])
    want_d = (want.astype(np.int64) + D).astype(np.int32)
    assert np.array_equal(gpu_gemm(dev, A, B, variant="padded"), want)
    assert np.array_equal(gpu_gemm(dev, A, B, D, variant="padded"), want_d)
    if m * n * k * batch >= 3 << 24:
        assert np.array_equal(gpu_gemm(dev, A, B, D), want_d)                # auto picks padded
    if batch == 1:
        plan = hg.make_plan(m, n, k, has_d=True, d_max_abs=1 << 20, variant="padded")
        Ct = torch.from_numpy(D.copy()).to(dev)
        hg.run(plan, torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev), Ct, out=Ct)
        assert np.array_equal(Ct.cpu().numpy(), want_d)                     # in place
    if m * n * k <= 1 << 30:
        assert np.array_equal(gpu_gemm(dev, A, B, variant="generic"), want)


def test_padded_variant_unaligned_pointers_and_pitches(dev):
    """A at an odd address with an odd pitch, B with a pitch that is not a
    multiple of 16, per-batch B: the copies read any layout."""
    batch, m, n, k = 2, 300, 250, 777
    lda, ldb = k + 3, n + 5
    rng = np.random.default_rng(9)
    A = rng.integers(-128, 128, (batch, m, lda), dtype=np.int8)
    B = rng.integers(-128, 128, (batch, k, ldb), dtype=np.int8)
    Abuf = torch.zeros(A.size + 1, dtype=torch.int8, device=dev)
    Abuf[1:] = torch.from_numpy(A.reshape(-1)).to(dev)
    Bt = torch.from_numpy(B).to(dev)
    C = torch.full((batch, m, n), INT32_MIN, dtype=torch.int32, device=dev)
    _lib.gemm_raw(Abuf.data_ptr() + 1, Bt.data_ptr(), None, C.data_ptr(), m, n, k, lda, ldb, n, n,
                  batch, m * lda, k * ldb, 0, m * n, "padded", 0, None)
    _lib.sync(None)
    got = C.cpu().numpy()
    for b in range(batch):
        assert np.array_equal(got[b], cref.gemm_i8(A[b, :, :k], B[b, :, :n], order="ikj")), b


@pytest.mark.parametrize("case", ["a_offset", "b_pitch", "b_stride"])
def test_padded_variant_copies_only_misaligned_operands(dev, case):
    """K and N multiples of 16 with one operand the vector kernels cannot read
    (A at an odd address, B with an odd pitch or batch stride): only that
    operand is copied and the product writes C itself, here with D in place
    and C at a pitch that is not a multiple of 16."""
    batch, m, n, k = 2, 200, 320, 512
    a_off = 1 if case == "a_offset" else 0
    ldb = n + 5 if case == "b_pitch" else n
    sb = k * ldb + (4 if case == "b_stride" else 0)
    ldc = n + 3
    rng = np.random.default_rng(11)
    A = rng.integers(-128, 128, (batch, m, k), dtype=np.int8)
    Bflat = rng.integers(-128, 128, batch * sb, dtype=np.int8)
    Bs = [Bflat[b * sb:b * sb + k * ldb].reshape(k, ldb)[:, :n] for b in range(batch)]
    D = rng.integers(-(1 << 20), (1 << 20) + 1, (batch, m, ldc), dtype=np.int32)
    Abuf = torch.zeros(A.size + 16, dtype=torch.int8, device=dev)
    Abuf[a_off:a_off + A.size] = torch.from_numpy(A.reshape(-1)).to(dev)
    Bt = torch.from_numpy(Bflat).to(dev)
    C = torch.from_numpy(D.copy()).to(dev)
    say("padded copies", case)
    _lib.gemm_raw(Abuf.data_ptr() + a_off, Bt.data_ptr(), C.data_ptr(), C.data_ptr(), m, n, k,
                  k, ldb, ldc, ldc, batch, m * k, sb, m * ldc, m * ldc, "padded", 0, None)
    _lib.sync(None)
    got = C.cpu().numpy()
    for b in range(batch):
        want = (cref.gemm_i8(A[b], Bs[b], order="ikj").astype(np.int64) + D[b, :, :n]).astype(np.int32)
        assert np.array_equal(got[b, :, :n], want), b
        assert np.array_equal(got[b, :, n:], D[b, :, n:]), b                 # past N untouched


# ---------------------------------------------------------------------------
# Seeded random sweep over every variant
# ---------------------------------------------------------------------------

def _random_case(rng, variant):
    """A random problem the variant accepts: shape, pitches, batch, shared B, D."""
    def dim(lo, hi, mult):
        return int(rng.integers(lo // mult, hi // mult + 1)) * mult
    mult = 1 if variant in ("generic", "padded") else 16
    m = int(rng.integers(1, 65)) if variant == "skinny" else int(rng.integers(1, 600))
    n, k = dim(16, 640, mult), dim(16, 1024, mult)
    pad_a = int(rng.integers(0, 3)) * (1 if mult == 1 else 16)
    pad_b = int(rng.integers(0, 3)) * (1 if mult == 1 else 16)
    batch = int(rng.choice([1, 1, 2, 3]))
    shared_b = bool(rng.integers(0, 2))
    has_d = bool(rng.integers(0, 2))
    in_place = has_d and bool(rng.integers(0, 2))
    return m, n, k, k + pad_a, n + pad_b, batch, shared_b, has_d, in_place


@pytest.mark.parametrize("variant", ["mfma_256x256", "mfma_256x128", "mfma_128x128", "skinny",
                                     "generic", "padded", "auto"])
def test_random_problems_match_the_oracle(dev, variant):
    rng = np.random.default_rng(sum(map(ord, variant)))
    for case in range(24 if variant != "generic" else 12):
        m, n, k, lda, ldb, batch, shared_b, has_d, in_place = _random_case(rng, variant)
        say("random", variant, case, (m, n, k, lda, ldb, batch, shared_b, has_d, in_place))
        A = rng.integers(-128, 128, (batch, m, lda), dtype=np.int8)
        B = rng.integers(-128, 128, (1 if shared_b else batch, k, ldb), dtype=np.int8)
        D = rng.integers(-(1 << 20), (1 << 20) + 1, (batch, m, n), dtype=np.int32)
        At, Bt = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
        Dt = torch.from_numpy(D).to(dev)
        C = Dt if in_place else torch.full((batch, m, n), INT32_MIN, dtype=torch.int32, device=dev)
        _lib.gemm_raw(At.data_ptr(), Bt.data_ptr(), Dt.data_ptr() if has_d else None, C.data_ptr(),
                      m, n, k, lda, ldb, n, n, batch, m * lda, 0 if shared_b else k * ldb,
                      m * n, m * n, variant, 0, None)
        _lib.sync(None)
        got = C.cpu().numpy()
        for b in range(batch):
            want = cref.gemm_i8(A[b, :, :k], B[0 if shared_b else b, :, :n],
                                D[b] if has_d else None, order="ikj")
            assert np.array_equal(got[b], want), (variant, case, b)


# Few long MFMA tiles: K runs as slices (batches of the same kernel) into a
# partial-sum workspace, added with D by the reduction kernel (from K = 8192
# also two slices over 65..128 tiles).
SPLIT_CASES = [("mfma_128x128", 128, 4096, 4096), ("mfma_128x128", 96, 2048, 2048),
               ("mfma_128x128", 100, 208, 2048), ("mfma_256x256", 256, 256, 8192),
               ("mfma_256x128", 256, 384, 4096), ("auto", 256, 1024, 4096),
               ("mfma_128x128", 768, 2048, 8192), ("mfma_256x128", 1280, 2048, 8192)]


@pytest.mark.parametrize("variant,m,n,k", SPLIT_CASES)
def test_mfma_k_split(dev, variant, m, n, k):
    name = variant if variant != "auto" else _lib.select_variant(m, n, k)[0]
    plan = hg.make_plan(m, n, k, variant=name)
    ks = hg.mfma_k_split(plan)
    say("mfma split", variant, m, n, k, "k slices", ks)
    assert ks > 1
    rng = np.random.default_rng(m + n + k)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = rng.integers(-(1 << 20), (1 << 20) + 1, (m, n), dtype=np.int32)
    assert np.array_equal(gpu_gemm(dev, A, B, variant=variant), go.gemm_i8_f64(A, B))
    At, Bt = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
    C = torch.from_numpy(D).to(dev)          # C = D + A.B in place
    _lib.gemm_raw(At.data_ptr(), Bt.data_ptr(), C.data_ptr(), C.data_ptr(), m, n, k, k, n, n, n,
                  1, 0, 0, 0, 0, variant, 0, None)
    _lib.sync(None)
    assert np.array_equal(C.cpu().numpy(), go.gemm_i8_f64(A, B, D))


def test_mfma_k_split_extremes_and_graph_replays(dev):
    m, n, k = 128, 256, 8192
    A = np.tile(np.array([-128, 127], np.int8), (m, k // 2))
    B = np.tile(np.array([[127], [-128]], np.int8), (k // 2, n))
    want = go.gemm_i8_f64(A, B)
    assert hg.mfma_k_split(hg.make_plan(m, n, k)) > 1
    At, Bt = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
    plan = hg.make_plan(m, n, k)
    s = torch.cuda.Stream(dev)
    outs = [torch.full((m, n), INT32_MIN, dtype=torch.int32, device=dev) for _ in range(3)]
    with torch.cuda.stream(s):
        hg.run(plan, At, Bt, out=outs[0], stream=s.cuda_stream)   # sizes the workspace
    s.synchronize()
    assert np.array_equal(outs[0].cpu().numpy(), want)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for C in outs[1:]:
            hg.run(plan, At, Bt, out=C, stream=s.cuda_stream)
    for rep in range(3):
        for C in outs[1:]:
            C.fill_(INT32_MIN)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for C in outs[1:]:
            assert np.array_equal(C.cpu().numpy(), want), rep

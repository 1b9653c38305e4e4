"""The 256x128 form of the persistent 16x16x64 kernel against the oracle,
through the C ABI (needs a gfx950 GPU).

mfma_256x128 problems with M >= 256, N >= 128, K a multiple of 256 and 16-byte
aligned C and D run persistently, one workgroup per CU, each wave computing a
128x64 block from direct-to-LDS slices and storing C through its LDS strip.
These cases check every output: one tile, a grid with several tiles per
workgroup, more tiles than CUs, D out of place and in place, D + A.B wrapping
past int32 through the raw C ABI, K split into slices summed by the reduction
kernel, unshared and shared-B batches, the int8 extremes, a row stride
wider than N, graph replays (unsplit and K-split), and ragged M and N (last
tiles moved back, shared rows and columns stored once). M below 256, N below
128 and K not a multiple of 256 stay on gemm_mfma_kernel<256, 128> (checked
here through the host model only).
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


def persistent(plan):
    lds, wgs = hg.required_resources(plan)
    return lds == hg.DMA16_LDS and wgs == min(hg.mfma_tiles(plan), hg.NUM_CUS)


# m, n, k, K slices
CASES = [
    (256, 128, 256, 1),       # one tile, one group of four slices
    (512, 384, 1024, 2),      # 6 tiles: K in 2 slices of 512
    (1280, 1152, 512, 1),     # 45 tiles
    (1536, 4096, 1024, 1),    # 192 tiles, the auto choice's region
    (2304, 2944, 256, 1),     # 207 tiles of one group each
    (4352, 2048, 512, 1),     # 272 tiles: more than one round on 256 CUs
    (512, 1024, 4096, 8),     # 16 tiles: K in 8 slices of 512
]


@pytest.mark.parametrize("m,n,k,ks", CASES)
def test_256x128_form_against_the_oracle(dev, m, n, k, ks):
    plan = hg.make_plan(m, n, k, variant="mfma_256x128")
    assert persistent(plan) and hg.mfma_k_split(plan) == ks
    st, _, v, native_ks, _ = _lib.gemm_check(m, n, k, k, n, n, n, variant="mfma_256x128")
    assert st == _lib.VT_OK and v == "mfma_256x128" and max(native_ks, 1) == ks
    rng = np.random.default_rng(m * 5 + n * 3 + k)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = rng.integers(-2**20, 2**20, (m, n), dtype=np.int32)
    At, Bt = to_dev(dev, A), to_dev(dev, B)
    say("256x128 form", m, n, k, ks)
    assert np.array_equal(hg.run(plan, At, Bt).cpu().numpy(), go.gemm_i8(A, B, None))
    plan_d = hg.make_plan(m, n, k, has_d=True, d_max_abs=2**20, variant="mfma_256x128")
    assert persistent(plan_d)
    want = go.gemm_i8(A, B, D)
    assert np.array_equal(hg.run(plan_d, At, Bt, to_dev(dev, D)).cpu().numpy(), want)
    C = to_dev(dev, D)
    assert np.array_equal(hg.run(plan_d, At, Bt, C, out=C).cpu().numpy(), want)
    # D near both ends of int32, so that D + A.B wraps (mod 2^32)
    Dw = np.where(rng.integers(0, 2, (m, n)) == 1, 2**31 - 7, -2**31 + 7).astype(np.int32)
    Cw = to_dev(dev, Dw)
    _lib.gemm_raw(At.data_ptr(), Bt.data_ptr(), Cw.data_ptr(), Cw.data_ptr(), m, n, k, k, n, n, n,
                  1, 0, 0, 0, 0, "mfma_256x128", 0, None)
    _lib.sync(None)
    assert np.array_equal(Cw.cpu().numpy(), go.gemm_i8(A, B, Dw))


@pytest.mark.parametrize("a,b", [(-128, -128), (-128, 127), (127, -128)])
def test_256x128_form_at_the_int8_extremes(dev, a, b):
    """Every product at (-128)^2 or -128 * 127, K = 2048: each sum at the end
    of its range."""
    m, n, k = 512, 1024, 2048
    plan = hg.make_plan(m, n, k, variant="mfma_256x128")
    assert persistent(plan)
    A, B = np.full((m, k), a, np.int8), np.full((k, n), b, np.int8)
    say("256x128 extremes", a, b)
    got = hg.run(plan, to_dev(dev, A), to_dev(dev, B)).cpu().numpy()
    assert np.array_equal(got, go.gemm_i8(A, B, None))


def test_256x128_form_on_batches(dev):
    """Unshared batches (each its own B, walked as tiles of one grid), and
    shared-B batches folded into one GEMM of stacked rows, with and without D."""
    m, n, k, batch = 512, 640, 768, 3
    rng = np.random.default_rng(11)
    A = rng.integers(-128, 128, (batch, m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (batch, k, n), dtype=np.int8)
    D = rng.integers(-2**20, 2**20, (batch, m, n), dtype=np.int32)
    At, Bt, Dt = to_dev(dev, A), to_dev(dev, B), to_dev(dev, D)
    assert persistent(hg.make_plan(m, n, k, batch=batch, variant="mfma_256x128"))
    C = torch.empty((batch, m, n), dtype=torch.int32, device=dev)
    Cd = torch.empty_like(C)
    say("256x128 batches")
    _lib.gemm_raw(At.data_ptr(), Bt.data_ptr(), None, C.data_ptr(), m, n, k, k, n, n, n,
                  batch, m * k, k * n, 0, m * n, "mfma_256x128", 0, None)
    _lib.gemm_raw(At.data_ptr(), Bt.data_ptr(), Dt.data_ptr(), Cd.data_ptr(), m, n, k, k, n, n, n,
                  batch, m * k, k * n, m * n, m * n, "mfma_256x128", 0, None)
    B0 = Bt[0].contiguous()
    Cs = torch.empty_like(C)
    _lib.gemm_raw(At.data_ptr(), B0.data_ptr(), Dt.data_ptr(), Cs.data_ptr(), m, n, k, k, n, n, n,
                  batch, m * k, 0, m * n, m * n, "mfma_256x128", 0, None)
    _lib.sync(None)
    for i in range(batch):
        assert np.array_equal(C[i].cpu().numpy(), go.gemm_i8(A[i], B[i], None)), i
        assert np.array_equal(Cd[i].cpu().numpy(), go.gemm_i8(A[i], B[i], D[i])), i
        assert np.array_equal(Cs[i].cpu().numpy(), go.gemm_i8(A[i], B[0], D[i])), i


def test_256x128_form_with_wide_rows(dev):
    """Row strides past N and K (a view into wider buffers): lda = K + 64,
    ldb = N + 128, ldc = ldd = N + 256, every one a multiple of 16 bytes; K
    below 1024, so the kernel itself writes C at that stride."""
    m, n, k = 768, 384, 768
    lda, ldb, ldc = k + 64, n + 128, n + 256
    rng = np.random.default_rng(12)
    Aw = rng.integers(-128, 128, (m, lda), dtype=np.int8)
    Bw = rng.integers(-128, 128, (k, ldb), dtype=np.int8)
    Dw = rng.integers(-2**20, 2**20, (m, ldc), dtype=np.int32)
    At, Bt, Dt = to_dev(dev, Aw), to_dev(dev, Bw), to_dev(dev, Dw)
    Ct = torch.full((m, ldc), -5, dtype=torch.int32, device=dev)
    say("256x128 wide rows")
    _lib.gemm_raw(At.data_ptr(), Bt.data_ptr(), Dt.data_ptr(), Ct.data_ptr(), m, n, k, lda, ldb, ldc,
                  ldc, 1, 0, 0, 0, 0, "mfma_256x128", 0, None)
    _lib.sync(None)
    got = Ct.cpu().numpy()
    assert np.array_equal(got[:, :n], go.gemm_i8(Aw[:, :k], Bw[:, :n], Dw[:, :n]))
    assert (got[:, n:] == -5).all()   # columns past N untouched


# m, n, k, K slices: the last tile row and/or column moved back to end at M
# or N, its shared rows and columns stored by the neighbour alone
RAGGED = [
    (300, 384, 1024, 2),      # M ragged (2 tile rows overlapping by 212), K split
    (2000, 4096, 512, 1),     # M ragged, 256 tiles
    (512, 4000, 768, 1),      # N ragged (32 columns past a whole tile)
    (1100, 1040, 2048, 4),    # both ragged, K split
    (256, 144, 256, 1),       # one tile row, N one tile plus 16 columns
]


@pytest.mark.parametrize("m,n,k,ks", RAGGED)
def test_256x128_form_on_ragged_shapes(dev, m, n, k, ks):
    """Moved-back last tiles: every element of C written once (a poisoned C
    outside M x N stays poisoned), with and without D, in place."""
    plan = hg.make_plan(m, n, k, variant="mfma_256x128")
    assert persistent(plan) and hg.mfma_k_split(plan) == ks
    rng = np.random.default_rng(m * 3 + n + k)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = rng.integers(-2**20, 2**20, (m, n), dtype=np.int32)
    At, Bt = to_dev(dev, A), to_dev(dev, B)
    say("256x128 ragged", m, n, k, ks)
    assert np.array_equal(hg.run(plan, At, Bt).cpu().numpy(), go.gemm_i8(A, B, None))
    plan_d = hg.make_plan(m, n, k, has_d=True, d_max_abs=2**20, variant="mfma_256x128")
    want = go.gemm_i8(A, B, D)
    assert np.array_equal(hg.run(plan_d, At, Bt, to_dev(dev, D)).cpu().numpy(), want)
    C = to_dev(dev, D)
    assert np.array_equal(hg.run(plan_d, At, Bt, C, out=C).cpu().numpy(), want)   # in place: D once
    # C inside a wider buffer: the columns past N keep their poison
    ldc = n + 64
    Cw = torch.full((m, ldc), -7, dtype=torch.int32, device=dev)
    _lib.gemm_raw(At.data_ptr(), Bt.data_ptr(), None, Cw.data_ptr(), m, n, k, k, n, ldc, ldc,
                  1, 0, 0, 0, 0, "mfma_256x128", 0, None)
    _lib.sync(None)
    got = Cw.cpu().numpy()
    assert np.array_equal(got[:, :n], go.gemm_i8(A, B, None))
    assert (got[:, n:] == -7).all()


def test_short_k_and_small_shapes_stay_on_the_tiled_kernel():
    """Host model: the 256x128 form needs M >= 256, N >= 128 and K % 256 == 0."""
    for m, n, k in ((200, 384, 1024), (512, 112, 1024), (512, 384, 320), (512, 384, 1088)):
        plan = hg.make_plan(m, n, k, variant="mfma_256x128")
        assert not persistent(plan), (m, n, k)


@pytest.mark.parametrize("m,n,k,ks", [(1536, 4096, 1024, 1), (512, 1024, 4096, 8)])
def test_256x128_form_in_graph_replays(dev, m, n, k, ks):
    """The form captured in a HIP graph, unsplit and with K slices through the
    stream's workspace (sized by an eager call first), C = D + A.B: every
    replay, with eager work and a poisoned C between replays, equals the
    eager result."""
    plan = hg.make_plan(m, n, k, has_d=True, d_max_abs=2**20, variant="mfma_256x128")
    assert persistent(plan) and hg.mfma_k_split(plan) == ks
    rng = np.random.default_rng(m + n + k)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = rng.integers(-2**20, 2**20, (m, n), dtype=np.int32)
    want = go.gemm_i8(A, B, D)
    At, Bt, Dt = to_dev(dev, A), to_dev(dev, B), to_dev(dev, D)
    s = torch.cuda.Stream(dev)
    outs = [torch.full((m, n), -2**31, dtype=torch.int32, device=dev) for _ in range(3)]
    say("256x128 graph", m, n, k, ks)
    with torch.cuda.stream(s):
        hg.run(plan, At, Bt, Dt, out=outs[0], stream=s.cuda_stream)
    s.synchronize()
    assert np.array_equal(outs[0].cpu().numpy(), want)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for C in outs[1:]:
            hg.run(plan, At, Bt, Dt, out=C, stream=s.cuda_stream)
    for rep in range(3):
        for C in outs[1:]:
            C.fill_(-2**31)
        scratch = torch.matmul(Dt[:64, :64].float(), Dt[:64, :64].float())   # eager work between
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert scratch.shape == (64, 64)
        for C in outs[1:]:
            assert np.array_equal(C.cpu().numpy(), want), rep

"""K-split decode sums finished inside the skinny kernel (needs a gfx950 GPU).

Up to 16 rows, vt_gemm_i8 finishes the K slices of the skinny (decode) kernel
in the kernel itself, through one 64-bit finishing word per two output
elements that every launch leaves zero (tests/test_fin_word.py models the
word). These tests call the C ABI and compare every output with the oracle:
row counts that take that path (odd ones, whose last word holds one row)
against the two-launch path's neighbours (17 rows, or a split whose count
does not fit the word), D and in place, batches, repeated calls and HIP graph
replays, so a word left nonzero by one launch would show in the next.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import gemm_oracle as go
from veritac_amd import _lib

pytestmark = pytest.mark.gpu

INT32_MIN = -2**31


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    lib = _lib.load_library()
    assert lib.vt_device_count() >= 1, "GPU visible but not gfx950"
    return torch.device("cuda", 0)


def say(*args):
    print(*args, flush=True)


def operands(rng, m, n, k, with_d, batch=1):
    shape_a = (batch, m, k) if batch > 1 else (m, k)
    A = rng.integers(-128, 128, shape_a, dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = (rng.integers(-2**31, 2**31, (batch, m, n) if batch > 1 else (m, n), dtype=np.int64)
         .astype(np.int32) if with_d else None)
    return A, B, D


def to_dev(dev, A, B, D):
    t = lambda x: None if x is None else torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
    return t(A), t(B), t(D)


def launch(At, Bt, Dt, C, k_split, stream=None):
    """C = D + A.B through vt_gemm_i8 (skinny variant) on device tensors, B
    shared by the batches."""
    batch = At.shape[0] if At.dim() == 3 else 1
    m, k = At.shape[-2:]
    n = Bt.shape[1]
    _lib.gemm_raw(At.data_ptr(), Bt.data_ptr(), None if Dt is None else Dt.data_ptr(),
                  C.data_ptr(), m, n, k, k, n, n, n, batch, m * k if batch > 1 else 0, 0,
                  m * n if (batch > 1 and Dt is not None) else 0, m * n if batch > 1 else 0,
                  "skinny", k_split, stream)


def run(dev, A, B, D, k_split, stream=None):
    At, Bt, Dt = to_dev(dev, A, B, D)
    C = torch.full(A.shape[:-1] + (B.shape[1],), INT32_MIN, dtype=torch.int32, device=dev)
    launch(At, Bt, Dt, C, k_split, stream)
    return C


def want(A, B, D):
    if A.ndim == 2:
        return go.gemm_i8(A, B, D)
    return np.stack([go.gemm_i8(A[i], B, None if D is None else D[i]) for i in range(A.shape[0])])


@pytest.mark.parametrize("m", [1, 2, 3, 5, 8, 13, 16, 17])
@pytest.mark.parametrize("k_split", [2, 3, 7, 64, 65])
def test_rows_and_splits(dev, m, k_split):
    """1-16 rows finish in the kernel, 17 take the reduction launch, and so
    does k_split 65 (65 slices of 128 rows: the count needs 7 bits beside two
    29-bit fields); N = 1040 leaves a partial last slab, K = 8256 a partial
    last slice."""
    rng = np.random.default_rng(100 * m + k_split)
    for with_d in (False, True):
        A, B, D = operands(rng, m, 1040, 8256, with_d)
        say("finish rows", m, "k_split", k_split, "D", with_d)
        C = run(dev, A, B, D, k_split)
        _lib.sync(None)
        assert np.array_equal(C.cpu().numpy(), want(A, B, D)), (m, k_split, with_d)


def test_in_place_and_wrap(dev):
    """C = C + A.B in place, with C near both ends of int32 so that the
    finished sum wraps (the contract's mod 2^32 result)."""
    rng = np.random.default_rng(7)
    m, n, k = 5, 2048, 4096
    A, B, _ = operands(rng, m, n, k, False)
    for base in (2**31 - 5, -2**31 + 5):
        D = np.full((m, n), base, np.int32)
        C = torch.from_numpy(D.copy()).to(dev)
        At, Bt = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
        say("finish in place", base)
        _lib.gemm_raw(At.data_ptr(), Bt.data_ptr(), C.data_ptr(), C.data_ptr(), m, n, k, k, n,
                      n, n, 1, 0, 0, 0, 0, "skinny", 4, None)
        _lib.sync(None)
        assert np.array_equal(C.cpu().numpy(), go.gemm_i8(A, B, D)), base


def test_batches_share_b(dev):
    rng = np.random.default_rng(8)
    A, B, D = operands(rng, 3, 1024, 4096, True, batch=5)
    say("finish batches")
    C = run(dev, A, B, D, 4)
    _lib.sync(None)
    assert np.array_equal(C.cpu().numpy(), want(A, B, D))


def test_repeated_calls_mixed_with_the_reduction_path(dev):
    """Finishing and two-launch calls in turn on one stream, each on new
    data: every result exact, so every launch left its words zero."""
    rng = np.random.default_rng(9)
    for it, (m, ks) in enumerate(((1, 4), (17, 4), (16, 4), (3, 5), (1, 4), (8, 2), (4, 64),
                                  (33, 4), (2, 3), (11, 7))):
        A, B, D = operands(rng, m, 1536, 4096, it % 2 == 1)
        say("finish repeat", it, m, ks)
        C = run(dev, A, B, D, ks)
        _lib.sync(None)
        assert np.array_equal(C.cpu().numpy(), want(A, B, D)), (it, m, ks)


def test_graph_replays(dev):
    """A finishing launch captured once (after the same call eagerly, so the
    stream has its words) and replayed with eager work and synchronisation
    between replays: every replay equals the oracle."""
    rng = np.random.default_rng(10)
    m, n, k = 2, 4096, 8192
    A, B, D = operands(rng, m, n, k, True)
    s = torch.cuda.Stream(device=dev)
    At, Bt, Dt = to_dev(dev, A, B, D)
    A2, B2, _ = operands(rng, 17, 1024, 4096, False)
    A2t, B2t, _ = to_dev(dev, A2, B2, None)
    C = torch.full((m, n), INT32_MIN, dtype=torch.int32, device=dev)
    C2 = torch.full((17, 1024), INT32_MIN, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    launch(At, Bt, Dt, C, 0, stream=s.cuda_stream)
    s.synchronize()
    assert np.array_equal(C.cpu().numpy(), want(A, B, D))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        launch(At, Bt, Dt, C, 0, stream=s.cuda_stream)
    for i in range(4):
        C.fill_(INT32_MIN)
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        s.synchronize()
        say("finish replay", i)
        assert np.array_equal(C.cpu().numpy(), want(A, B, D)), i
        # eager work on the same stream between replays, through the other path
        C2.fill_(INT32_MIN)
        torch.cuda.synchronize()
        launch(A2t, B2t, None, C2, 4, stream=s.cuda_stream)
        s.synchronize()
        assert np.array_equal(C2.cpu().numpy(), want(A2, B2, None)), i


def test_two_streams_at_once(dev):
    """Each stream has its own finishing words: finishing launches on two
    streams, enqueued together and left to overlap, are both exact."""
    rng = np.random.default_rng(11)
    s1, s2 = torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)
    jobs = []
    for s in (s1, s2):
        A, B, D = operands(rng, 3, 4096, 8192, True)
        At, Bt, Dt = to_dev(dev, A, B, D)
        C = torch.full((3, 4096), INT32_MIN, dtype=torch.int32, device=dev)
        jobs.append((s, A, B, D, At, Bt, Dt, C))
    torch.cuda.synchronize()
    for rep in range(3):
        for s, A, B, D, At, Bt, Dt, C in jobs:
            C.fill_(INT32_MIN)
        torch.cuda.synchronize()
        for s, A, B, D, At, Bt, Dt, C in jobs:
            launch(At, Bt, Dt, C, 4, stream=s.cuda_stream)
        torch.cuda.synchronize()
        say("finish two streams", rep)
        for s, A, B, D, At, Bt, Dt, C in jobs:
            assert np.array_equal(C.cpu().numpy(), want(A, B, D)), rep

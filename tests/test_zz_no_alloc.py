"""vt_gemm_i8_noalloc (needs a gfx950 GPU): the same results as vt_gemm_i8,
with its scratch from the library's static array instead of allocations.

Each case makes two calls in a row through the C ABI, the second smaller,
and compares both outputs bit for bit with vt_gemm_i8 on the same operands
(outputs poisoned with INT32_MIN first), and with the CPU oracle. The cases
are the ones that take scratch: the decode kernel's K-split partial sums,
the padded variant's copies (with an inner K split as well), and the K-split
partial sums of the rows, or the columns, a 256x256 problem runs on 128x128
tiles after its whole tiles.
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
    assert _lib.load_library().vt_device_count() >= 1, "GPU visible but not gfx950"
    return torch.device("cuda", 0)


def say(*args):
    print(*args, flush=True)


def operands(dev, m, n, k, seed, with_d):
    rng = np.random.default_rng(seed)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    D = rng.integers(-2**20, 2**20, (m, n), dtype=np.int32) if with_d else None
    t = lambda x: None if x is None else torch.from_numpy(x).to(dev)   # noqa: E731
    return (A, B, D), (t(A), t(B), t(D))


def call(fn, dev, At, Bt, Dt, m, n, k, variant="auto", k_split=0, stream=None):
    C = torch.full((m, n), INT32_MIN, dtype=torch.int32, device=dev)
    fn(At.data_ptr(), Bt.data_ptr(), None if Dt is None else Dt.data_ptr(), C.data_ptr(),
       m, n, k, k, n, n, n, 1, 0, 0, 0, 0, variant, k_split, stream)
    return C


def scratch_bytes(m, n, k, variant="auto", k_split=0, with_d=False):
    st, reason, v, _, ws = _lib.gemm_check(m, n, k, k, n, n, n, has_d=with_d, variant=variant,
                                           k_split=k_split)
    assert st == 0, reason
    return v, ws


# (first call, second smaller call): m, n, k, variant, k_split, D
PAIRS = [
    ("decode k-split", (16, 14336, 4096, "auto", 0, False), (8, 2048, 1024, "auto", 0, True)),
    ("decode explicit split", (16, 4096, 8192, "skinny", 16, True), (1, 1024, 2048, "skinny", 3, False)),
    ("padded", (1000, 1000, 1000, "auto", 0, True), (300, 500, 700, "padded", 0, False)),
    ("padded inner k-split", (16, 2047, 4095, "padded", 0, False), (5, 999, 1001, "padded", 0, True)),
    # whole 256-row tiles on the persistent kernel, the last 40 (52) rows on
    # 64x64 tiles with K in 2 slices: 1.25 MiB, then 832 KiB of scratch
    ("256x256 row split", (4136, 4096, 1024, "mfma_256x256", 0, True),
     (8244, 2048, 1024, "mfma_256x256", 0, False)),
    # whole 256-column tiles on the persistent kernel, the last 16 columns on
    # 64x64 tiles with K in 4 (then 2) slices: 1 MiB, then 512 KiB of scratch
    ("256x256 column split", (4096, 4112, 4096, "mfma_256x256", 0, True),
     (4096, 4112, 1024, "mfma_256x256", 0, False)),
    # the persistent kernel's 256x128 form with K in 8 (then 4) slices as
    # batches into the partials: 16 MiB, then 13.5 MiB of scratch
    ("256x128 form k-split", (512, 1024, 4096, "mfma_256x128", 0, True),
     (768, 1152, 2048, "mfma_256x128", 0, False)),
]


@pytest.mark.parametrize("name,first,second", PAIRS, ids=[p[0] for p in PAIRS])
def test_noalloc_equals_gemm_i8_on_two_calls(dev, name, first, second):
    for i, (m, n, k, variant, ks, with_d) in enumerate((first, second)):
        v, ws = scratch_bytes(m, n, k, variant, ks, with_d)
        say(name, "call", i, (m, n, k, variant, ks, with_d), "->", v, ws, "bytes of scratch")
        assert 0 < ws <= _lib.NOALLOC_SCRATCH_BYTES
        (A, B, D), (At, Bt, Dt) = operands(dev, m, n, k, 100 * i + len(name), with_d)
        got = call(_lib.gemm_noalloc_raw, dev, At, Bt, Dt, m, n, k, variant, ks)
        want = call(_lib.gemm_raw, dev, At, Bt, Dt, m, n, k, variant, ks)
        torch.cuda.synchronize()
        got, want = got.cpu().numpy(), want.cpu().numpy()
        assert np.array_equal(got, want), (name, i)
        assert np.array_equal(got, go.gemm_i8(A, B, D)), (name, i)


def test_noalloc_without_scratch_and_in_place(dev):
    """Calls that take no scratch (MFMA, VALU) and in-place C = C + A.B."""
    for m, n, k in ((256, 512, 320), (64, 64, 64), (33, 48, 80)):
        (A, B, D), (At, Bt, Dt) = operands(dev, m, n, k, m, True)
        C = Dt.clone()
        _lib.gemm_noalloc_raw(At.data_ptr(), Bt.data_ptr(), C.data_ptr(), C.data_ptr(),
                              m, n, k, k, n, n, n)
        torch.cuda.synchronize()
        assert np.array_equal(C.cpu().numpy(), go.gemm_i8(A, B, D)), (m, n, k)


def test_noalloc_refuses_calls_beyond_the_scratch_array(dev):
    """A padded call whose copies exceed the array is refused before any
    launch: the output keeps its poison."""
    m = n = k = 3000 - 1
    v, ws = scratch_bytes(m, n, k)
    assert v == "padded" and ws > _lib.NOALLOC_SCRATCH_BYTES
    _, (At, Bt, _) = operands(dev, m, n, k, 5, False)
    C = torch.full((m, n), INT32_MIN, dtype=torch.int32, device=dev)
    with pytest.raises(_lib.HipGemmError) as exc:
        _lib.gemm_noalloc_raw(At.data_ptr(), Bt.data_ptr(), None, C.data_ptr(),
                              m, n, k, k, n, n, n)
    assert exc.value.code == _lib.VT_EUNSUPPORTED and "static scratch array" in str(exc.value)
    torch.cuda.synchronize()
    assert bool((C == INT32_MIN).all())


def test_noalloc_first_call_on_a_stream_under_graph_capture(dev):
    """The caller it is for: a first call on a fresh stream, inside HIP
    graph capture, needing scratch (vt_gemm_i8 refuses that). Every replay,
    with eager work and synchronization between replays, equals the oracle."""
    m, n, k = 16, 4096, 8192
    _, ws = scratch_bytes(m, n, k)
    assert ws > 0
    (A, B, _), (At, Bt, _) = operands(dev, m, n, k, 9, False)
    want = go.gemm_i8(A, B)
    s = torch.cuda.Stream(device=dev)
    C = torch.empty((m, n), dtype=torch.int32, device=dev)
    # the library's first use of the device (its set-up) happens eagerly
    _lib.gemm_noalloc_raw(At.data_ptr(), Bt.data_ptr(), None, C.data_ptr(), m, n, k, k, n, n, n)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        _lib.gemm_noalloc_raw(At.data_ptr(), Bt.data_ptr(), None, C.data_ptr(),
                              m, n, k, k, n, n, n, stream=s.cuda_stream)
    for i in range(3):
        C.fill_(INT32_MIN)
        with torch.cuda.stream(s):
            g.replay()
        s.synchronize()
        assert np.array_equal(C.cpu().numpy(), want), "replay %d" % i

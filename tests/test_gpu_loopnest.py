"""Emitted loop-nest kernels on the GPU (needs a gfx950 GPU).

Every kernel is compiled by hipRTC through the native library and launched
through vt_rtc_launch. Results are compared with the sequential oracle
interpreter and with closed forms; the status word must be 0 except in the
tests that plant an out-of-range index or a division by zero, where it must
name exactly that event and the kernel must not touch memory outside its
buffers.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from loopnest_tactics import reorder, tile
from test_loopnest_host import DISJOINT_CASES
from oracle import gemm_oracle as go
from oracle import loopnest_interp as li
from veritac_amd import _lib
from veritac_amd.specializations.hip_gemm import loopnest as ln

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    assert _lib.load_library().vt_device_count() >= 1, "GPU visible but not gfx950"
    return torch.device("cuda", 0)


def say(*args):
    print(*args, flush=True)


def lit(v):
    return {"tag": "lit", "val": v}


def var(n):
    return {"tag": "var", "name": n}


def rd(buf, *idx):
    return {"tag": "bufRead", "buf": buf, "indices": list(idx)}


def wr(buf, idx, val):
    return {"tag": "bufWrite", "buf": buf, "indices": list(idx), "val": val}


def loop(v, hi, body, ann="none"):
    return {"tag": "loop", "var": v, "lo": lit(0), "hi": lit(hi), "ann": ann, "body": body}


NESTS = {
    "naive": lambda M, K, N: ln.matmul_stmt(M, K, N),
    "tiled": lambda M, K, N: tile(tile(ln.matmul_stmt(M, K, N), "i0", 4), "i1", 8),
    "k_outer": lambda M, K, N: reorder(reorder(ln.matmul_stmt(M, K, N), "i1", "i2"), "i0", "i2"),
    "tiled_k": lambda M, K, N: tile(ln.matmul_stmt(M, K, N), "i2", 4),
}


@pytest.mark.parametrize("nest", sorted(NESTS))
@pytest.mark.parametrize("shape", [(8, 12, 16), (40, 64, 24), (64, 256, 48)])
def test_int8_gemm_nests_are_exact(dev, nest, shape):
    M, K, N = shape
    say("loopnest", nest, shape)
    rng = np.random.default_rng(M + K + N)
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B = rng.integers(-128, 128, (K, N), dtype=np.int8)
    D = rng.integers(-2**20, 2**20, (M, N), dtype=np.int32)
    stmt = NESTS[nest](M, K, N)
    k = ln.LoopNestKernel(stmt, {"A": {"dtype": "int8", "shape": (M, K)},
                                 "B": {"dtype": "int8", "shape": (K, N)},
                                 "C": {"dtype": "int32", "shape": (M, N)}})
    t = {"A": torch.from_numpy(A.reshape(-1)).to(dev), "B": torch.from_numpy(B.reshape(-1)).to(dev),
         "C": torch.from_numpy(D.reshape(-1).copy()).to(dev)}
    status = k(t)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    got = t["C"].cpu().numpy().reshape(M, N)
    assert np.array_equal(got, go.gemm_i8(A, B, D))
    if M * N * K <= 8 * 12 * 16:
        bufs = {"A": A.reshape(-1).copy(), "B": B.reshape(-1).copy(), "C": D.reshape(-1).copy()}
        li.run(stmt, bufs, {"A": (M, K), "B": (K, N), "C": (M, N)})
        assert np.array_equal(got.reshape(-1), bufs["C"])


@pytest.mark.parametrize("nest", ["naive", "tiled", "k_outer"])
def test_reference_benchmark_protocol(dev, nest):
    """benchmark_matmul: the reference runner's inputs, layout and keys."""
    M, K, N = 32, 48, 64
    res = ln.benchmark_matmul(NESTS[nest](M, K, N), M, K, N, num_runs=3)
    say(nest, {k: res[k] for k in ("gpu_time_ms", "correct", "status", "mapped_loops")})
    assert res["correct"] and res["status"] == 0
    A = np.fromfunction(lambda i, k: (i * K + k) % 7, (M, K), dtype=np.int64)
    B = np.fromfunction(lambda k, j: (k * N + j) % 5, (K, N), dtype=np.int64)
    C = A @ B
    assert res["gpu_first_values"] == [float(C[0, 0]), float(C[1, 0]), float(C[M - 1, 0]),
                                       float(C[M - 1, N - 1])]
    assert res["gpu_time_ms"] > 0


def test_out_of_range_index_is_contained_and_reported(dev):
    n = 64
    stmt = loop("i", n, wr("Y", [{"tag": "add", "left": var("i"), "right": lit(1)}], rd("X", var("i"))),
                "parallel")
    k = ln.LoopNestKernel(stmt, {"X": {"dtype": "int32", "shape": (n,)},
                                 "Y": {"dtype": "int32", "shape": (n,)}})
    assert k.info["mapped"] == ["i"]
    x = torch.arange(n, dtype=torch.int32, device=dev)
    guard = torch.full((n + 16,), -7, dtype=torch.int32, device=dev)
    y = guard[:n]
    status = k({"X": x, "Y": y})
    torch.cuda.synchronize()
    assert int(status.item()) == ln.STATUS_RANGE
    out = guard.cpu().numpy()
    assert out[0] == -7 and np.array_equal(out[1:n], np.arange(n - 1))
    assert np.all(out[n:] == -7)                  # nothing written past Y


def test_integer_division_by_zero_is_reported(dev):
    n = 16
    den = {"tag": "add", "left": var("i"), "right": lit(-3)}
    stmt = loop("i", n, wr("Y", [var("i")], {"tag": "div", "left": rd("X", var("i")), "right": den}))
    k = ln.LoopNestKernel(stmt, {"X": {"dtype": "int64", "shape": (n,)},
                                 "Y": {"dtype": "int64", "shape": (n,)}})
    x_np = np.arange(n, dtype=np.int64) * -37 + 11
    x = torch.from_numpy(x_np).to(dev)
    y = torch.zeros(n, dtype=torch.int64, device=dev)
    status = k({"X": x, "Y": y})
    torch.cuda.synchronize()
    assert int(status.item()) == ln.STATUS_DIV0
    got = y.cpu().numpy()
    for i in range(n):
        if i == 3:
            assert got[i] == 0
        else:
            a, b = int(x_np[i]), i - 3
            q = abs(a) // abs(b)
            assert got[i] == (q if (a >= 0) == (b >= 0) else -q), i


def test_private_buffers_and_float_arithmetic(dev):
    n = 256
    body = {"tag": "alloc", "buf": "t", "shape": [lit(2)], "body": {
        "tag": "seq",
        "s1": wr("t", [lit(0)], {"tag": "mul", "left": rd("X", var("i")), "right": rd("X", var("i"))}),
        "s2": {"tag": "seq",
               "s1": wr("t", [lit(1)], {"tag": "mod", "left": rd("t", lit(0)), "right": lit(7)}),
               "s2": wr("Y", [var("i")], {"tag": "add", "left": rd("t", lit(0)),
                                          "right": {"tag": "div", "left": rd("t", lit(1)),
                                                    "right": lit(4)}})}}}
    stmt = loop("i", n, body, "parallel")
    decl = {"X": {"dtype": "float64", "shape": (n,)}, "Y": {"dtype": "float64", "shape": (n,)}}
    k = ln.LoopNestKernel(stmt, decl)
    assert k.info["mapped"] == ["i"]
    x_np = np.linspace(-3.0, 5.0, n)
    x = torch.from_numpy(x_np).to(dev)
    y = torch.zeros(n, dtype=torch.float64, device=dev)
    assert int(k({"X": x, "Y": y}).item()) == 0
    torch.cuda.synchronize()
    bufs = {"X": x_np.copy(), "Y": np.zeros(n)}
    li.run(stmt, bufs, {"X": (n,), "Y": (n,)})
    assert np.array_equal(y.cpu().numpy(), bufs["Y"])   # no FMA contraction: same rounding


def test_kernel_reuse_across_calls(dev):
    M, K, N = 16, 32, 16
    k = ln.LoopNestKernel(ln.matmul_stmt(M, K, N), {"A": {"dtype": "int8", "shape": (M, K)},
                                                   "B": {"dtype": "int8", "shape": (K, N)},
                                                   "C": {"dtype": "int32", "shape": (M, N)}})
    for seed in range(3):
        rng = np.random.default_rng(seed)
        A = rng.integers(-128, 128, (M, K), dtype=np.int8)
        B = rng.integers(-128, 128, (K, N), dtype=np.int8)
        C = torch.zeros(M * N, dtype=torch.int32, device=dev)
        st = k({"A": torch.from_numpy(A.reshape(-1)).to(dev),
                "B": torch.from_numpy(B.reshape(-1)).to(dev), "C": C})
        torch.cuda.synchronize()
        assert int(st.item()) == 0
        assert np.array_equal(C.cpu().numpy().reshape(M, N), go.gemm_i8(A, B))


# ---------------------------------------------------------------------------
# Mapping only where threads own disjoint cells; other edge cases
# ---------------------------------------------------------------------------

def _run_vs_interp(dev, stmt, decl, inputs, stream=None):
    """Launch the nest, then compare every buffer with the sequential oracle."""
    k = ln.LoopNestKernel(stmt, decl)
    t = {b: torch.from_numpy(inputs[b].copy()).to(dev) for b in decl}
    status = k(t, stream=stream)
    torch.cuda.synchronize()
    bufs = {b: inputs[b].copy() for b in decl}
    li.run(stmt, bufs, {b: decl[b]["shape"] for b in decl})
    for b in decl:
        assert np.array_equal(t[b].cpu().numpy(), bufs[b]), b
    return k, int(status.item())


def _inputs(decl, seed):
    rng = np.random.default_rng(seed)
    out = {}
    for b, d in decl.items():
        n = int(np.prod(d["shape"]))
        if d["dtype"] in ("float32", "float64"):
            out[b] = rng.uniform(-4, 4, n).astype(d["dtype"])
        else:
            out[b] = rng.integers(-100, 100, n).astype(d["dtype"])
    return out


GPU_DISJOINT = [c for c in DISJOINT_CASES if c[0] not in ("row_spill", "data_bound")]


@pytest.mark.parametrize("name,stmt,decl,want", GPU_DISJOINT, ids=[c[0] for c in GPU_DISJOINT])
def test_order_dependent_nests_match_the_sequential_oracle(dev, name, stmt, decl, want):
    say("disjoint", name, want)
    k, st = _run_vs_interp(dev, stmt, decl, _inputs(decl, len(name)))
    assert st == 0 and k.info["mapped"] == want


def test_loop_bound_is_reevaluated_every_iteration(dev):
    stmt = {"tag": "loop", "var": "i", "lo": lit(0), "hi": rd("Y", lit(0)), "ann": "none",
            "body": wr("Y", [lit(0)], {"tag": "add", "left": rd("Y", lit(0)), "right": lit(-1)})}
    k, st = _run_vs_interp(dev, stmt, {"Y": {"dtype": "int32", "shape": (1,)}},
                           {"Y": np.array([5], np.int32)})
    assert st == 0 and k.info["mapped"] == []


def test_iteration_cap_stops_a_thread_and_reports_it(dev):
    """for (i = 0; i < Y[0]; i++) Y[0] = Y[0] - 1 from 10^6 runs 500000
    iterations; with a cap of 1000 the thread stops after its 1000th
    iteration, leaves Y[0] = 10^6 - 1000 and sets STATUS_ITERATIONS."""
    stmt = {"tag": "loop", "var": "i", "lo": lit(0), "hi": rd("Y", lit(0)), "ann": "none",
            "body": wr("Y", [lit(0)], {"tag": "add", "left": rd("Y", lit(0)), "right": lit(-1)})}
    k = ln.LoopNestKernel(stmt, {"Y": {"dtype": "int32", "shape": (1,)}}, max_iterations=1000)
    y = torch.tensor([10**6], dtype=torch.int32, device=dev)
    status = k({"Y": y})
    torch.cuda.synchronize()
    assert int(status.item()) == ln.STATUS_ITERATIONS
    assert int(y.item()) == 10**6 - 1000


def test_each_store_typed_by_its_own_buffers_and_int64_wraps(dev):
    mul = lambda a, b: {"tag": "mul", "left": a, "right": b}      # noqa: E731
    stmt = {"tag": "seq",
            "s1": wr("Z", [lit(0)], mul(rd("W", lit(0)), rd("W", lit(0)))),
            "s2": {"tag": "seq", "s1": wr("F", [lit(0)], mul(rd("W", lit(1)), lit(3))),
                   "s2": wr("Z", [lit(1)], mul(rd("W", lit(1)), rd("W", lit(1))))}}
    decl = {"W": {"dtype": "int64", "shape": (2,)}, "Z": {"dtype": "int64", "shape": (2,)},
            "F": {"dtype": "float64", "shape": (1,)}}
    w = np.array([2**40 + 3, 2**31 + 1], np.int64)
    k, st = _run_vs_interp(dev, stmt, decl, {"W": w, "Z": np.zeros(2, np.int64),
                                             "F": np.zeros(1)})
    assert st == 0


def test_floating_index_truncates_toward_zero(dev):
    stmt = loop("i", 2, wr("Y", [var("i")], rd("S", rd("X", var("i")))))
    decl = {"X": {"dtype": "float64", "shape": (2,)}, "S": {"dtype": "int64", "shape": (3,)},
            "Y": {"dtype": "int64", "shape": (2,)}}
    _, st = _run_vs_interp(dev, stmt, decl, {"X": np.array([2.7, -0.5]),
                                             "S": np.array([10, 20, 30], np.int64),
                                             "Y": np.zeros(2, np.int64)})
    assert st == 0


def test_caller_stream_is_ordered_after_the_current_one(dev):
    M, K, N = 64, 96, 80
    decl = {"A": {"dtype": "int8", "shape": (M, K)}, "B": {"dtype": "int8", "shape": (K, N)},
            "C": {"dtype": "int32", "shape": (M, N)}}
    k = ln.LoopNestKernel(ln.matmul_stmt(M, K, N), decl)
    rng = np.random.default_rng(5)
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B = rng.integers(-128, 128, (K, N), dtype=np.int8)
    side = torch.cuda.Stream(device=dev)
    for rep in range(3):
        t = {"A": torch.from_numpy(A.reshape(-1)).to(dev), "B": torch.from_numpy(B.reshape(-1)).to(dev),
             "C": torch.full((M * N,), 7, dtype=torch.int32, device=dev)}
        side.wait_stream(torch.cuda.current_stream(dev))      # inputs are filled on the current stream
        status = k(t, stream=side.cuda_stream)
        side.synchronize()
        assert int(status.item()) == 0
        assert np.array_equal(t["C"].cpu().numpy().reshape(M, N),
                              go.gemm_i8(A, B, np.full((M, N), 7, np.int32)))
    res = ln.benchmark_matmul(ln.matmul_stmt(24, 40, 56), 24, 40, 56, num_runs=3,
                              stream=side.cuda_stream)
    assert res["correct"] and res["status"] == 0 and res["gpu_time_ms"] > 0


def test_empty_loop_launches_nothing(dev):
    k = ln.LoopNestKernel(loop("i", 0, wr("Y", [var("i")], lit(1))),
                          {"Y": {"dtype": "int32", "shape": (4,)}})
    y = torch.full((4,), -3, dtype=torch.int32, device=dev)
    assert int(k({"Y": y}).item()) == 0
    assert y.cpu().tolist() == [-3] * 4


def test_nest_without_buffers_reports_division_by_zero(dev):
    stmt = {"tag": "loop", "var": "i", "lo": lit(0),
            "hi": {"tag": "div", "left": lit(1), "right": lit(0)}, "ann": "none", "body": {"tag": "skip"}}
    k = ln.LoopNestKernel(stmt, {})
    assert k.info["params"] == [] and k.info["threads"] == 1
    status = k({})
    torch.cuda.synchronize()
    assert int(status.item()) == ln.STATUS_DIV0

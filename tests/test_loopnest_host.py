"""Loop-nest emitter on the CPU: parsing and its refusals, the independence
analysis and thread mapping, the oracle interpreter against closed forms,
and hipRTC compilation of emitted kernels (no device needed)."""
import numpy as np
import pytest
import torch

from loopnest_tactics import annotate, reorder, tile
from oracle import loopnest_interp as li
from veritac_amd import HipGemmError
from veritac_amd.specializations.hip_gemm import loopnest as ln


def lit(v):
    return {"tag": "lit", "val": v}


def var(n):
    return {"tag": "var", "name": n}


def rd(buf, *idx):
    return {"tag": "bufRead", "buf": buf, "indices": list(idx)}


def wr(buf, idx, val):
    return {"tag": "bufWrite", "buf": buf, "indices": list(idx), "val": val}


def loop(v, hi, body, ann="none", lo=0):
    return {"tag": "loop", "var": v, "lo": lit(lo), "hi": lit(hi), "ann": ann, "body": body}


def gemm_decl(M, K, N, dt=("int8", "int8", "int32")):
    return {"A": {"dtype": dt[0], "shape": (M, K)}, "B": {"dtype": dt[1], "shape": (K, N)},
            "C": {"dtype": dt[2], "shape": (M, N)}}


def interp_gemm(stmt, A, B, D):
    M, K = A.shape
    N = B.shape[1]
    bufs = {"A": A.reshape(-1).copy(), "B": B.reshape(-1).copy(), "C": D.reshape(-1).copy()}
    li.run(stmt, bufs, {"A": (M, K), "B": (K, N), "C": (M, N)})
    return bufs["C"].reshape(M, N)


NESTS = {
    "naive": lambda M, K, N: ln.matmul_stmt(M, K, N),
    "tiled": lambda M, K, N: tile(tile(ln.matmul_stmt(M, K, N), "i0", 4), "i1", 8),
    "k_outer": lambda M, K, N: reorder(reorder(ln.matmul_stmt(M, K, N), "i1", "i2"), "i0", "i2"),
    "tiled_k": lambda M, K, N: tile(ln.matmul_stmt(M, K, N), "i2", 4),
}


# ---------------------------------------------------------------------------
# The oracle interpreter, pinned by closed forms
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("nest", sorted(NESTS))
def test_interpreter_gives_d_plus_ab(nest):
    M, K, N = 8, 12, 16
    rng = np.random.default_rng(1)
    A = rng.integers(-128, 128, (M, K), dtype=np.int8)
    B = rng.integers(-128, 128, (K, N), dtype=np.int8)
    D = rng.integers(-2**20, 2**20, (M, N), dtype=np.int32)
    want = (D.astype(np.int64) + A.astype(np.int64) @ B.astype(np.int64)).astype(np.int32)
    assert np.array_equal(interp_gemm(NESTS[nest](M, K, N), A, B, D), want)


def test_interpreter_reference_layout_and_runner_inputs():
    M, K, N = 3, 4, 5
    A = np.fromfunction(lambda i, k: (i * K + k) % 7, (M, K), dtype=np.int64).astype(float)
    B = np.fromfunction(lambda k, j: (k * N + j) % 5, (K, N), dtype=np.int64).astype(float)
    flat = {name: np.zeros((r - 1) * 1000 + c) for name, (r, c) in
            (("A", (M, K)), ("B", (K, N)), ("C", (M, N)))}
    for name, mat in (("A", A), ("B", B)):
        for r in range(mat.shape[0]):
            flat[name][r * 1000:r * 1000 + mat.shape[1]] = mat[r]
    li.run(ln.matmul_stmt(M, K, N), flat, layout="reference")
    got = np.array([[flat["C"][i * 1000 + j] for j in range(N)] for i in range(M)])
    assert np.array_equal(got, A @ B)


def test_interpreter_c_division_and_bounds():
    x = np.array([-7, 7, -8, 9], np.int64)
    y = np.zeros(4, np.int64)
    stmt = loop("i", 4, wr("Y", [var("i")], {"tag": "div", "left": rd("X", var("i")), "right": lit(2)}))
    li.run(stmt, {"X": x, "Y": y}, {"X": (4,), "Y": (4,)})
    assert y.tolist() == [-3, 3, -4, 4]          # truncation toward zero, as in C
    stmt = loop("i", 4, wr("Y", [var("i")], {"tag": "mod", "left": rd("X", var("i")), "right": lit(3)}))
    li.run(stmt, {"X": x, "Y": y}, {"X": (4,), "Y": (4,)})
    assert y.tolist() == [-1, 1, -2, 0]
    with pytest.raises(IndexError):
        li.run(loop("i", 5, wr("Y", [var("i")], lit(1))), {"Y": y}, {"Y": (4,)})


# ---------------------------------------------------------------------------
# Parsing and refusals
# ---------------------------------------------------------------------------

def test_parse_every_tag():
    stmt = {"tag": "seq", "s1": {"tag": "skip"},
            "s2": {"tag": "alloc", "buf": "t", "shape": [lit(2)],
                   "body": loop("i", 2, wr("t", [var("i")], {"tag": "mod", "left": var("i"),
                                                             "right": lit(2)}), "unrolled")}}
    ir = ln.parse_stmt(stmt)
    assert ir[0] == "seq" and ir[1][0] == ("skip",) and ir[1][1][0] == "alloc"


@pytest.mark.parametrize("bad", [
    {"tag": "loopy"},
    {"tag": "bufWrite", "buf": "C", "indices": [], "val": {"tag": "pow"}},
    loop("i", 2, wr("C", [var("i")], lit(1)), ann="gpu"),
    loop("i", 2, wr("vt_status", [var("i")], lit(1))),
    loop("int", 2, wr("C", [var("int")], lit(1))),
    loop("i", 2, wr("C", [var("j")], lit(1))),                       # unbound
    loop("i", 2, loop("i", 2, wr("C", [var("i")], lit(1)))),         # shadowing
    loop("i", 2, wr("C", [var("i")], {"tag": "lit", "val": 1.5})),
    loop("i", 2, wr("Z", [var("i")], lit(1))),                       # undeclared buffer
])
def test_malformed_nests_rejected(bad):
    with pytest.raises(ln.LoopNestError):
        ln.emit_kernel(bad, {"C": {"dtype": "int32", "shape": (2,)}})


def test_declaration_errors():
    with pytest.raises(ln.LoopNestError):
        ln.emit_kernel(ln.matmul_stmt(2, 2, 2), gemm_decl(2, 2, 2, ("int8", "int8", "int128")))
    with pytest.raises(ln.LoopNestError):
        ln.emit_kernel(ln.matmul_stmt(2, 2, 2), gemm_decl(2, 2, 2), layout="strided")
    with pytest.raises(ln.LoopNestError):   # 3 indices into a 2-D dense buffer
        ln.emit_kernel(loop("i", 2, wr("C", [var("i"), lit(0), lit(0)], lit(1))),
                       {"C": {"dtype": "int32", "shape": (2, 2)}})
    assert issubclass(ln.LoopNestError, HipGemmError)


# ---------------------------------------------------------------------------
# Independence and thread mapping
# ---------------------------------------------------------------------------

def test_mapping_of_the_matmul_nests():
    decl = gemm_decl(8, 12, 16)
    info = ln.emit_kernel(NESTS["naive"](8, 12, 16), decl)
    assert info["mapped"] == ["i0", "i1"] and info["threads"] == 8 * 16
    assert info["grid"] == (1, 1, 1) and info["params"] == ["A", "B", "C"]
    assert info["written"] == ["C"]
    info = ln.emit_kernel(NESTS["tiled"](8, 12, 16), decl)
    assert info["mapped"] == ["i0_outer", "i0_inner", "i1_outer", "i1_inner"]
    info = ln.emit_kernel(NESTS["k_outer"](8, 12, 16), decl)
    assert info["mapped"] == ["i0", "i1"]                  # k stays sequential per thread
    assert "for (long long i2 = 0LL; i2 < 12LL; ++i2)" in info["source"]
    info = ln.emit_kernel(NESTS["tiled_k"](8, 12, 16), decl)
    assert info["mapped"] == ["i0", "i1"]


def test_reduction_annotations_are_suppressed():
    nest = annotate(ln.matmul_stmt(4, 4, 4), "i2", "parallel")
    info = ln.emit_kernel(nest, gemm_decl(4, 4, 4))
    assert "i2" not in info["mapped"]
    assert any("parallel suppressed on i2" in n for n in info["notes"])
    assert "// parallel suppressed on i2" in info["source"]


def test_independence_needs_one_index_list():
    # C[i] = C[i] + X[i, j]: j is a reduction
    red = loop("i", 4, loop("j", 3, wr("C", [var("i")], {"tag": "add", "left": rd("C", var("i")),
                                                          "right": rd("X", var("i"), var("j"))}),
                            ann="vectorize"))
    info = ln.emit_kernel(red, {"C": {"dtype": "int32", "shape": (4,)},
                                "X": {"dtype": "int32", "shape": (4, 3)}})
    assert info["mapped"] == ["i"] and any("vectorize suppressed on j" in n for n in info["notes"])
    # Y[i+1] = Y[i] + 1 reads another iteration's cell: nothing is mapped
    shift = loop("i", 3, wr("Y", [{"tag": "add", "left": var("i"), "right": lit(1)}],
                            {"tag": "add", "left": rd("Y", var("i")), "right": lit(1)}), "parallel")
    info = ln.emit_kernel(shift, {"Y": {"dtype": "int32", "shape": (4,)}})
    assert info["mapped"] == [] and info["threads"] == 1
    assert not ln.independent("i", ln.parse_stmt(shift)[5])
    # a buffer alloc'd inside the loop is private to the iteration
    priv = loop("i", 4, {"tag": "alloc", "buf": "t", "shape": [lit(1)],
                         "body": {"tag": "seq", "s1": wr("t", [lit(0)], rd("X", var("i"), lit(0))),
                                  "s2": wr("C", [var("i")], rd("t", lit(0)))}})
    info = ln.emit_kernel(priv, {"C": {"dtype": "int32", "shape": (4,)},
                                 "X": {"dtype": "int32", "shape": (4, 3)}})
    assert info["mapped"] == ["i"]


# ---------------------------------------------------------------------------
# Emitted kernels compile (hipRTC needs no device)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("nest", sorted(NESTS))
@pytest.mark.parametrize("layout", ["dense", "reference"])
def test_emitted_kernels_compile(nest, layout):
    dt = ("int8", "int8", "int32") if layout == "dense" else ("float64",) * 3
    k = ln.LoopNestKernel(NESTS[nest](8, 12, 16), gemm_decl(8, 12, 16, dt), layout=layout)
    assert k.program.code_size > 1000
    assert "vt_idx(" in k.source and "atomicOr" in k.source


def test_compile_errors_are_reported():
    from veritac_amd import _lib
    with pytest.raises(HipGemmError, match="hiprtcCompileProgram"):
        _lib.RtcProgram('extern "C" __global__ void k() { undefined_thing(); }', "k")


def test_kernel_call_refuses_bad_tensors_before_launch():
    k = ln.LoopNestKernel(ln.matmul_stmt(4, 4, 4), gemm_decl(4, 4, 4))
    ok = {"A": torch.zeros(16, dtype=torch.int8), "B": torch.zeros(16, dtype=torch.int8),
          "C": torch.zeros(16, dtype=torch.int32)}
    with pytest.raises(ln.LoopNestError, match="GPU only"):
        k(ok)
    with pytest.raises(ln.LoopNestError, match="must be int32"):
        k(dict(ok, C=torch.zeros(16, dtype=torch.int64)))
    with pytest.raises(ln.LoopNestError, match="needs 16"):
        k(dict(ok, C=torch.zeros(15, dtype=torch.int32)))
    with pytest.raises(ln.LoopNestError, match="missing tensor"):
        k({"A": ok["A"], "B": ok["B"]})

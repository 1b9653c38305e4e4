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


# ---------------------------------------------------------------------------
# Disjointness: threads of the mapped loops never share a cell
# ---------------------------------------------------------------------------

def add(a, b):
    return {"tag": "add", "left": a, "right": b}


def mul(a, b):
    return {"tag": "mul", "left": a, "right": b}


def bump(buf, *idx):
    """buf[idx] = buf[idx] * 2 + 1: one index list, order-dependent value."""
    return wr(buf, list(idx), add(mul(rd(buf, *idx), lit(2)), lit(1)))


def y_decl(n, extra=None):
    decl = {"Y": {"dtype": "int32", "shape": (n,)}}
    decl.update(extra or {})
    return decl


def _copy_and_reduce(row):
    """Y[row*i + k] = X[i, k]; W[i] = W[i] + X[i, k]."""
    return {"tag": "seq",
            "s1": wr("Y", [add(mul(var("i"), lit(row)), var("k"))], rd("X", var("i"), var("k"))),
            "s2": wr("W", [var("i")], add(rd("W", var("i")), rd("X", var("i"), var("k"))))}


X34 = {"X": {"dtype": "int32", "shape": (3, 4)}}
X48 = {"X": {"dtype": "int32", "shape": (4, 8)}}

DISJOINT_CASES = [
    # Y[i + j]: both loops mention the cell, and (0,1), (1,0) collide
    ("sum_of_mapped", loop("i", 4, loop("j", 4, bump("Y", add(var("i"), var("j")))), "parallel"),
     y_decl(8), []),
    # Y[j % 2]: not affine
    ("modulo", loop("j", 4, bump("Y", {"tag": "mod", "left": var("j"), "right": lit(2)})),
     y_decl(2), []),
    # Y[2i + j]: j < 2 separates, j < 3 does not
    ("radix_ok", loop("i", 4, loop("j", 2, bump("Y", add(mul(var("i"), lit(2)), var("j"))))),
     y_decl(8), ["i", "j"]),
    ("radix_overlap", loop("i", 4, loop("j", 3, bump("Y", add(mul(lit(2), var("i")), var("j"))))),
     y_decl(9), []),
    # C[i, j] with j running past the row aliases the next row
    ("row_spill", loop("i", 4, loop("j", 8, bump("Y", var("i"), var("j")))),
     {"Y": {"dtype": "int32", "shape": (4, 4)}}, []),
    ("row_exact", loop("i", 4, loop("j", 4, bump("Y", var("i"), var("j")))),
     {"Y": {"dtype": "int32", "shape": (4, 4)}}, ["i", "j"]),
    # a time loop outside: t stays sequential, j is mapped
    ("time_loop", loop("t", 3, loop("j", 4, wr("Y", [var("j")], add(rd("Y", var("j")),
                                                                   rd("X", var("t"), var("j")))))),
     y_decl(4, X34), ["j"]),
    # a sequential inner loop (it also reduces into W[i]) in the index:
    # 8i + k separates k < 8, 4i + k does not
    ("inner_digit", loop("i", 4, loop("k", 8, _copy_and_reduce(8), "unrolled")),
     y_decl(32, dict(X48, W={"dtype": "int32", "shape": (4,)})), ["i"]),
    ("inner_overlap", loop("i", 4, loop("k", 8, _copy_and_reduce(4))),
     y_decl(32, dict(X48, W={"dtype": "int32", "shape": (4,)})), []),
    # triangular inner loop: k < i + 1 <= 4, so 4i + k separates
    ("triangular", loop("i", 4, {"tag": "loop", "var": "k", "lo": lit(0), "hi": add(var("i"), lit(1)),
                                 "ann": "none", "body": bump("Y", add(mul(var("i"), lit(4)), var("k")))}),
     y_decl(16), ["i"]),
    # a bound read from memory leaves k's range unknown
    ("data_bound", loop("i", 4, {"tag": "loop", "var": "k", "lo": lit(0), "hi": rd("X", var("i"), lit(0)),
                                 "ann": "none", "body": bump("Y", add(mul(var("i"), lit(4)), var("k")))}),
     y_decl(16, X48), []),
    # negative coefficient: Y[7 - i]
    ("reversed", loop("i", 8, bump("Y", add(lit(7), mul(lit(-1), var("i")))), "parallel"),
     y_decl(8), ["i"]),
]


@pytest.mark.parametrize("name,stmt,decl,want", DISJOINT_CASES, ids=[c[0] for c in DISJOINT_CASES])
def test_mapping_only_where_threads_own_disjoint_cells(name, stmt, decl, want):
    info = ln.emit_kernel(stmt, decl)
    assert info["mapped"] == want
    if want:        # nothing mapped: nothing to enumerate (and bounds may read memory)
        _assert_disjoint_by_enumeration(ln.parse_stmt(stmt), set(want), decl, "dense")


def test_suppression_note_names_the_collision():
    stmt = loop("i", 4, loop("j", 4, bump("Y", add(var("i"), var("j"))), "vectorize"), "parallel")
    notes = ln.emit_kernel(stmt, y_decl(8))["notes"]
    assert "parallel suppressed on i: iterations may write the same cell" in notes
    assert "vectorize suppressed on j: iterations may write the same cell" in notes


def _points(stmt, env, out):
    """Every (env, buffer, flat cell) a nest's writes touch, by running its
    loops (bounds over variables and literals only)."""
    kind = stmt[0]
    if kind == "loop":
        lo = _value(stmt[2], env)
        v = lo
        while v < _value(stmt[3], env):
            _points(stmt[5], dict(env, **{stmt[1]: v}), out)
            v += 1
    elif kind == "seq":
        for s in stmt[1]:
            _points(s, env, out)
    elif kind == "write":
        out.append((env, stmt[1], tuple(_value(i, env) for i in stmt[2])))
    return out


def _value(e, env):
    if e[0] == "lit":
        return e[1]
    if e[0] == "var":
        return env[e[1]]
    a, b = _value(e[1], env), _value(e[2], env)
    if e[0] == "add":
        return a + b
    if e[0] == "mul":
        return a * b
    assert b != 0
    q = abs(a) // abs(b) * (1 if (a >= 0) == (b >= 0) else -1)
    return q if e[0] == "div" else a - b * q


def _assert_disjoint_by_enumeration(stmt, mapped, decl, layout):
    """Brute force: no cell is written by two different mapped tuples."""
    owner = {}
    for env, buf, idx in _points(stmt, {}, []):
        shape = decl[buf]["shape"]
        flat = 0
        for d, i in enumerate(idx):
            flat = flat * (ln.REFERENCE_STRIDE if layout == "reference" else shape[d]) + i
        key = tuple(sorted((v, env[v]) for v in mapped))
        assert owner.setdefault((buf, flat), key) == key, (buf, flat, owner[(buf, flat)], key)


def test_disjointness_is_sound_on_random_affine_nests():
    """threads_disjoint never accepts a mapped set whose threads share a
    cell: random 3-deep nests with affine (sometimes triangular) bounds and
    affine 1-D or 2-D indices, every subset of the loops checked against
    enumeration of every iteration point."""
    import itertools
    rng = np.random.default_rng(12345)
    names = ("a", "b", "c")
    accepted = rejected = 0
    for trial in range(400):
        ext = [int(x) for x in rng.integers(1, 5, 3)]
        coef = [[int(x) for x in rng.integers(-4, 5, 3)] for _ in range(2)]
        dims = int(rng.integers(1, 3))
        triangular = bool(rng.integers(0, 3) == 0)
        idx = []
        for d in range(dims):
            e = lit(0)
            for n, c in zip(names, coef[d]):
                if c:
                    e = add(e, mul(lit(c), var(n)))
            idx.append(e)
        body = bump("Y", *idx)
        inner_hi = add(var("b"), lit(1)) if triangular else lit(ext[2])
        stmt_json = loop("a", ext[0], loop("b", ext[1], {"tag": "loop", "var": "c", "lo": lit(0),
                                                         "hi": inner_hi, "ann": "none",
                                                         "body": body}))
        stmt = ln.parse_stmt(stmt_json)
        # shift indices to be non-negative and size Y to hold every cell
        pts = _points(stmt, {}, [])
        lows = [min(p[2][d] for p in pts) for d in range(dims)]
        highs = [max(p[2][d] for p in pts) for d in range(dims)]
        idx = [add(i, lit(-lo)) for i, lo in zip(idx, lows)]
        stmt_json = loop("a", ext[0], loop("b", ext[1], {"tag": "loop", "var": "c", "lo": lit(0),
                                                         "hi": inner_hi, "ann": "none",
                                                         "body": bump("Y", *idx)}))
        stmt = ln.parse_stmt(stmt_json)
        decl = {"Y": {"dtype": "int32", "shape": tuple(h - lo + 1 for h, lo in zip(highs, lows))}}
        for r in range(1, 4):
            for subset in itertools.combinations(range(3), r):
                if triangular and 2 in subset:
                    continue                       # mapped loops need constant bounds
                mapped = {names[s]: ext[s] for s in subset}
                if ln.threads_disjoint(stmt, mapped, decl):
                    accepted += 1
                    _assert_disjoint_by_enumeration(stmt, set(mapped), decl, "dense")
                else:
                    rejected += 1
        got = ln.emit_kernel(stmt_json, decl)["mapped"]
        _assert_disjoint_by_enumeration(stmt, set(got), decl, "dense")
    assert accepted > 200 and rejected > 200       # both verdicts exercised


# ---------------------------------------------------------------------------
# Other edge cases of the emitter and the interpreter
# ---------------------------------------------------------------------------

def test_literals_must_fit_int64():
    for v in (2**63, -2**63, 10**30):
        with pytest.raises(ln.LoopNestError, match="lit value"):
            ln.parse_expr(lit(v))
    assert ln.parse_expr(lit(2**63 - 1)) == ("lit", 2**63 - 1)


def test_empty_mapped_loop_emits_no_zero_divisor():
    k = ln.LoopNestKernel(loop("i", 0, wr("Y", [var("i")], lit(1))), y_decl(4))
    assert k.info["threads"] == 0 and k.info["mapped"] == ["i"]
    assert "% 0LL" not in k.source and "/= 0LL" not in k.source


def test_written_buffers_may_not_overlap_others():
    k = ln.LoopNestKernel(loop("i", 4, wr("Y", [var("i")], rd("X", var("i")))),
                          {"X": {"dtype": "int32", "shape": (4,)}, "Y": {"dtype": "int32", "shape": (4,)}})
    base = torch.zeros(8, dtype=torch.int32)
    with pytest.raises(ln.LoopNestError, match="overlaps"):
        k({"X": base[0:4], "Y": base[2:6]})
    with pytest.raises(ln.LoopNestError, match="GPU only"):   # disjoint views pass that check
        k({"X": base[0:4], "Y": base[4:8]})


def test_interpreter_reevaluates_loop_bounds_like_c():
    # for (i = 0; i < Y[0]; i++) Y[0] = Y[0] - 1;  from 5: i=0 (5->4), 1 (4->3), 2 (3->2), stop
    stmt = {"tag": "loop", "var": "i", "lo": lit(0), "hi": rd("Y", lit(0)), "ann": "none",
            "body": wr("Y", [lit(0)], add(rd("Y", lit(0)), lit(-1)))}
    y = np.array([5], np.int64)
    li.run(stmt, {"Y": y}, {"Y": (1,)})
    assert y[0] == 2


def test_interpreter_types_each_store_by_its_own_buffers():
    # Z = W * W stays exact in integers although a float64 buffer exists
    w = np.array([2**31 + 1], np.int64)
    z = np.zeros(1, np.int64)
    f = np.zeros(1, np.float64)
    stmt = {"tag": "seq", "s1": wr("Z", [lit(0)], mul(rd("W", lit(0)), rd("W", lit(0)))),
            "s2": wr("F", [lit(0)], mul(rd("W", lit(0)), lit(3)))}
    li.run(stmt, {"W": w, "Z": z, "F": f}, {"W": (1,), "Z": (1,), "F": (1,)})
    assert int(z[0]) == (2**31 + 1) ** 2 and f[0] == 3.0 * (2**31 + 1)
    # a floating value used as an index truncates toward zero
    x = np.array([2.7, -0.5])
    src = np.array([10, 20, 30], np.int64)
    y = np.zeros(2, np.int64)
    li.run(loop("i", 2, wr("Y", [var("i")], rd("S", rd("X", var("i"))))),
           {"X": x, "S": src, "Y": y}, {"X": (2,), "S": (3,), "Y": (2,)})
    assert y.tolist() == [30, 10]


def test_sequential_work_per_thread_is_bounded():
    """A nest whose threads would run more than the cap of sequential
    iterations is refused when emitted, with no device involved."""
    one = {"Y": {"dtype": "int64", "shape": (1,)}}
    # Y[0] += 1, 2^62 times: no loop is independent, so one thread runs it all
    runaway = loop("i", 2**62, wr("Y", [lit(0)], add(rd("Y", lit(0)), lit(1))))
    with pytest.raises(ln.LoopNestError, match="beyond the cap"):
        ln.emit_kernel(runaway, one)
    # nested: 2^14 x 2^13 sequential iterations exceed 2^26 only through the product
    nested = loop("i", 2**14, loop("j", 2**13, wr("Y", [lit(0)], add(rd("Y", lit(0)), lit(1)))))
    with pytest.raises(ln.LoopNestError, match="beyond the cap"):
        ln.emit_kernel(nested, one)
    # the reference's largest nest, 1000^3: (i, j) are threads, 1000 per thread
    info = ln.emit_kernel(ln.matmul_stmt(1000, 1000, 1000),
                          {"A": {"dtype": "float64", "shape": (1000, 1000)},
                           "B": {"dtype": "float64", "shape": (1000, 1000)},
                           "C": {"dtype": "float64", "shape": (1000, 1000)}}, layout="reference")
    assert ln.thread_iterations(ln.parse_stmt(ln.matmul_stmt(1000, 1000, 1000)),
                                set(info["mapped"]), ln._var_ranges(
                                    ln.parse_stmt(ln.matmul_stmt(1000, 1000, 1000)), {})) == 1000
    assert "vt_iters" not in info["source"]
    # a triangular nest is bounded through its outer variable's range
    tri = loop("i", 3000, {"tag": "loop", "var": "j", "lo": lit(0), "hi": var("i"), "ann": "none",
                           "body": wr("Y", [lit(0)], add(rd("Y", lit(0)), lit(1)))})
    assert ln.thread_iterations(ln.parse_stmt(tri), set(), ln._var_ranges(ln.parse_stmt(tri), {})) \
        == 3000 * (1 + 2999)
    ln.emit_kernel(tri, one)
    with pytest.raises(ln.LoopNestError):
        ln.emit_kernel(tri, one, max_iterations=1000)
    with pytest.raises(ln.LoopNestError, match="max_iterations"):
        ln.emit_kernel(tri, one, max_iterations=0)


def test_memory_bounds_are_counted_at_run_time():
    """A bound that reads memory cannot be bounded statically: every
    sequential loop then counts its iterations against the cap in the
    emitted kernel, which stops the thread and sets STATUS_ITERATIONS."""
    stmt = {"tag": "loop", "var": "i", "lo": lit(0), "hi": rd("Y", lit(0)), "ann": "none",
            "body": wr("Y", [lit(0)], add(rd("Y", lit(0)), lit(-1)))}
    info = ln.emit_kernel(stmt, {"Y": {"dtype": "int32", "shape": (1,)}}, max_iterations=777)
    src = info["source"]
    assert "unsigned long long vt_iters = 0;" in src
    assert "if (++vt_iters > 777ULL) { atomicOr(vt_status, %d); return; }" \
        % ln.STATUS_ITERATIONS in src
    assert any("counted" in n for n in info["notes"])

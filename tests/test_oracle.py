"""Pins of the CPU oracle (oracle/) before it is trusted as the checker.

Each oracle function is checked against data or mathematics that a plausible
mistake would break: the reference's recorded Spike outputs (24 full-output
vectors, independent of the reference's Python), the reference's hand
known-answer tests, brute force, exact float64 BLAS, K-tiling invariance and
two's-complement wrap-around; a planted mistake must fail the golden check.
"""
import numpy as np
import pytest

from oracle import cref
from oracle import gemm_oracle as go
from conftest import decode_cout


def _case_arrays(run, mode):
    m, n, k = run["plan"]["m"], run["plan"]["n"], run["plan"]["k"]
    a, b = go.fill_inputs(mode, m * k, k * n)
    A = np.frombuffer(a, dtype=np.int8).reshape(m, k)
    B = np.frombuffer(b, dtype=np.int8).reshape(k, n)
    return A, B


def test_golden_fixture_complete(golden):
    runs = golden["runs"]
    assert len(runs) == 8
    assert golden["modes"] == ["zeros", "extrema", "lcg"]
    shapes = sorted((r["plan"]["m"], r["plan"]["n"], r["plan"]["k"]) for r in runs)
    assert (16, 32, 48) in shapes and (48, 16, 32) in shapes and (32, 16, 32) in shapes


@pytest.mark.parametrize("mode", ["zeros", "extrema", "lcg"])
def test_reference_matmul_matches_spike_outputs(golden, mode):
    for run in golden["runs"]:
        m, n, k = run["plan"]["m"], run["plan"]["n"], run["plan"]["k"]
        a, b = go.fill_inputs(mode, m * k, k * n)
        assert go.reference_matmul(a, b, m, n, k) == decode_cout(run["cout"][mode]), run["name"]


@pytest.mark.parametrize("mode", ["zeros", "extrema", "lcg"])
def test_numpy_and_c_oracles_match_spike_outputs(golden, mode):
    for run in golden["runs"]:
        A, B = _case_arrays(run, mode)
        want = np.array(decode_cout(run["cout"][mode]), dtype=np.int32).reshape(A.shape[0], B.shape[1])
        assert np.array_equal(go.gemm_i8_int64(A, B), want), run["name"]
        assert np.array_equal(go.gemm_i8_f64(A, B), want), run["name"]
        assert np.array_equal(cref.gemm_i8(A, B), want), run["name"]
        assert np.array_equal(cref.gemm_i8(A, B, order="ikj"), want), run["name"]
        assert np.array_equal(go.gemm_i8_ktiled(A, B, k_tile=16), want), run["name"]
        # scalar_matmul on flat lists of the same int8 values
        flatA = [int(v) for v in A.reshape(-1)]
        flatB = [int(v) for v in B.reshape(-1)]
        assert go.scalar_matmul(flatA, flatB, A.shape[0], B.shape[1], A.shape[1]) == want.reshape(-1).tolist()


def test_baseline_and_reuse_b_schedules_agree(golden):
    by_shape = {}
    for run in golden["runs"]:
        p = run["plan"]
        by_shape.setdefault((p["m"], p["n"], p["k"]), []).append(run)
    pairs = [v for v in by_shape.values() if len(v) == 2]
    assert len(pairs) >= 3
    for a, b in pairs:
        assert a["cout"] == b["cout"]


def test_planted_mistake_fails_golden(golden):
    """An oracle that drops the K-tile partial sum (overwrites instead of
    accumulating after the first 16-wide tile) must disagree with Spike."""
    def dropped_partial(A, B):
        return go.gemm_i8_int64(A[:, -16:], B[-16:, :])   # only the last K tile
    mism = 0
    for run in golden["runs"]:
        if run["plan"]["k"] <= 16:
            continue
        A, B = _case_arrays(run, "lcg")
        want = np.array(decode_cout(run["cout"]["lcg"]), dtype=np.int32).reshape(A.shape[0], B.shape[1])
        mism += not np.array_equal(dropped_partial(A, B), want)
    assert mism >= 3


def test_hand_known_answers():
    # run_raw_spike tests: zeros, 2x2 extrema, mixed sign (test_gemmini_raw_spike.py:176-194)
    assert go.reference_matmul(bytes(4), bytes(4), 2, 2, 2) == [0, 0, 0, 0]
    a, b = go.fill_inputs("extrema", 4, 4)
    assert list(a) == [0x80, 0x7F, 0x80, 0x7F] and list(b) == [0x7F, 0x80, 0x7F, 0x80]
    assert go.reference_matmul(a, b, 2, 2, 2) == [-127, 128, -127, 128]
    assert go.reference_matmul(bytes([1, 2, 3, 4]), bytes([5, 256 - 6, 7, 256 - 8]), 2, 2, 2) == \
        [19, -22, 43, -50]
    # cpu_gemm 2x2 known answer (tests/test_matmul.py:64-70)
    A = np.array([[1, 2], [3, 4]], np.int8)
    B = np.array([[5, 6], [7, 8]], np.int8)
    want = np.array([[19, 22], [43, 50]], np.int32)
    assert np.array_equal(go.gemm_i8(A, B), want)
    assert np.array_equal(cref.gemm_i8(A, B), want)
    assert go.scalar_matmul([1, 2, 3, 4], [5, 6, 7, 8], 2, 2, 2) == [19, 22, 43, 50]


def test_lcg8_first_values_and_spread():
    s = go.lcg8_stream(64)
    # x1 = (0x12345678 * 1103515245 + 12345) mod 2^32 = 0x0b719151, so the first
    # byte is 0x71 (the full stream is pinned by the lcg Spike vectors).
    assert s[0] == 0x71
    assert len(set(s)) > 1 and all(0 <= v < 256 for v in s)


def test_deterministic_inputs_relation_and_c_twin():
    # value = byte - 128 of the same state sequence (backend.py:583-593 vs 738-746)
    m, n, k, seed = 5, 7, 9, 917
    A, B = go.deterministic_inputs(m, n, k, seed, "lcg")
    stream = go.lcg8_stream(m * k + k * n, seed)
    assert A + B == [v - 128 for v in stream]
    ca, cb = cref.lcg_fill(seed, m * k, k * n)
    assert A == ca.tolist() and B == cb.tolist()
    for mode, (va, vb) in {"max": (127, 127), "minmax": (-128, 127), "min": (-128, -128),
                           "zero": (0, 0)}.items():
        A, B = go.deterministic_inputs(2, 3, 4, 0, mode)
        assert set(A) == {va} and set(B) == {vb} and len(A) == 8 and len(B) == 12
    with pytest.raises(ValueError):
        go.deterministic_inputs(1, 1, 1, 0, "bogus")


def test_brute_force_tiny_and_blas_agree():
    rng = np.random.default_rng(1)
    for (m, n, k) in [(1, 1, 1), (3, 5, 7), (4, 16, 33), (9, 2, 64)]:
        A = rng.integers(-128, 128, (m, k), dtype=np.int8)
        B = rng.integers(-128, 128, (k, n), dtype=np.int8)
        D = rng.integers(-(1 << 20), 1 << 20, (m, n), dtype=np.int32)
        brute = np.zeros((m, n), np.int64)
        for i in range(m):
            for j in range(n):
                brute[i, j] = sum(int(A[i, t]) * int(B[t, j]) for t in range(k)) + int(D[i, j])
        brute = brute.astype(np.int32)
        assert np.array_equal(go.gemm_i8_int64(A, B, D), brute)
        assert np.array_equal(go.gemm_i8_f64(A, B, D), brute)
        assert np.array_equal(cref.gemm_i8(A, B, D), brute)
        assert np.array_equal(cref.gemm_i8(A, B, D, order="ikj"), brute)
        for kt in (1, 16, 64):
            assert np.array_equal(go.gemm_i8_ktiled(A, B, D, k_tile=kt), brute)


def test_extremes_near_overflow_bound():
    # all -128 x -128 over K = 131071: 131071 * 16384 = 2^31 - 16384 fits;
    # K = 131072 reaches 2^31 and the scalar oracle raises (backend.py:575-577)
    k = 131071
    A = np.full((1, k), -128, np.int8)
    B = np.full((k, 1), -128, np.int8)
    assert int(go.gemm_i8_int64(A, B)[0, 0]) == k * 16384
    assert int(cref.gemm_i8(A, B)[0, 0]) == k * 16384
    with pytest.raises(go.OracleOverflow):
        go.scalar_matmul([-128] * 131072, [-128] * 131072, 1, 1, 131072)


def test_int32_wraparound_matches_signed32():
    # Word.lean:31: results are taken mod 2^32 (two's complement)
    A = np.array([[1]], np.int8)
    B = np.array([[1]], np.int8)
    D = np.array([[2**31 - 1]], np.int32)
    assert int(go.gemm_i8_int64(A, B, D)[0, 0]) == -2**31
    assert int(cref.gemm_i8(A, B, D)[0, 0]) == -2**31
    assert int(go.gemm_i8_ktiled(A, B, D, k_tile=1)[0, 0]) == -2**31


def test_batched_broadcast_equals_per_batch():
    rng = np.random.default_rng(3)
    A = rng.integers(-128, 128, (4, 8, 32), dtype=np.int8)
    B = rng.integers(-128, 128, (32, 16), dtype=np.int8)
    C = go.gemm_i8(A, B)
    for b in range(4):
        assert np.array_equal(C[b], cref.gemm_i8(A[b], B))


def test_deterministic_inputs_match_reference_vectors():
    """deterministic_inputs and scalar_matmul against vectors the reference's
    own functions produced (tests/golden/make_lcg_vectors.py), in every mode:
    the oracle's restatement, its C twin and the product's generator."""
    import json
    import os
    from veritac_amd.specializations.hip_gemm import inputs
    path = os.path.join(os.path.dirname(__file__), "golden", "lcg_inputs.json")
    with open(path) as fh:
        cases = json.load(fh)["cases"]
    assert len(cases) == 10
    assert {c["mode"] for c in cases} == {"lcg", "max", "minmax", "min", "zero"}
    for c in cases:
        m, n, k, seed, mode = c["m"], c["n"], c["k"], c["seed"], c["mode"]
        A, B = go.deterministic_inputs(m, n, k, seed, mode)
        assert (A, B) == (c["A"], c["B"]), (m, n, k, seed, mode)
        An, Bn = inputs.deterministic_inputs(m, n, k, seed, mode)
        assert An.reshape(-1).tolist() == c["A"] and Bn.reshape(-1).tolist() == c["B"]
        assert go.scalar_matmul(c["A"], c["B"], m, n, k) == c["C"]
        assert go.gemm_i8(An, Bn).reshape(-1).tolist() == c["C"]
        if mode == "lcg":
            ca, cb = cref.lcg_fill(seed, m * k, k * n)
            assert ca.tolist() == c["A"] and cb.tolist() == c["B"]


def test_reference_vectors_pin_the_byte_mapping():
    """The fixture tells byte - 128 from the two's-complement reading of the
    same bytes (the Spike harness's mapping): a planted swap must fail it."""
    import json
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "lcg_inputs.json")
    with open(path) as fh:
        c = json.load(fh)["cases"][2]
    stream = go.lcg8_stream(c["m"] * c["k"] + c["k"] * c["n"], c["seed"])
    assert [b - 128 for b in stream[:c["m"] * c["k"]]] == c["A"]
    assert [go.to_int8(b) for b in stream[:c["m"] * c["k"]]] != c["A"]


def _oracle_builds():
    builds = ["default", "O2"]
    if cref.host_has_avx512():
        builds.append("v4")
    return builds


@pytest.mark.parametrize("variant", _oracle_builds())
def test_every_oracle_build_matches_the_spike_outputs_and_brute_force(golden, variant):
    """The -O2 (reference runner flags) and -O3 builds of the C restatement
    compute the same function: the recorded Spike outputs and a brute-force
    sum with D and a K that is not a multiple of 16."""
    for run in golden["runs"]:
        A, B = _case_arrays(run, "lcg")
        want = np.array(decode_cout(run["cout"]["lcg"]), dtype=np.int32).reshape(A.shape[0], B.shape[1])
        for order in ("ijk", "ikj"):
            assert np.array_equal(cref.gemm_i8(A, B, order=order, variant=variant), want), run["name"]
    rng = np.random.default_rng(7)
    A = rng.integers(-128, 128, (5, 37), dtype=np.int8)
    B = rng.integers(-128, 128, (37, 11), dtype=np.int8)
    D = rng.integers(-2**31, 2**31, (5, 11), dtype=np.int64).astype(np.int32)
    brute = [[(int(D[i, j]) + sum(int(A[i, t]) * int(B[t, j]) for t in range(37)) + 2**31) % 2**32 - 2**31
              for j in range(11)] for i in range(5)]
    for order in ("ijk", "ikj"):
        assert cref.gemm_i8(A, B, D, order=order, variant=variant).tolist() == brute


def test_unavailable_builds_refuse_to_load():
    with pytest.raises(ValueError):
        cref.load(variant="O7")
    if not cref.host_has_avx512():
        with pytest.raises(RuntimeError, match="AVX-512"):
            cref.load(variant="v4")


def _stride1000(mat):
    rows, cols = mat.shape
    flat = np.zeros((rows - 1) * 1000 + cols)
    for r in range(rows):
        flat[r * 1000:r * 1000 + cols] = mat[r]
    return flat


@pytest.mark.parametrize("variant", ["default", "O2"])
def test_f64_stride1000_nest_is_the_reference_runner_gemm(variant):
    """The reference's CPU GEMM (naive nest, stride-1000 double buffers) on the
    runner's own inputs A = (i*K+k)%7, B = (k*N+j)%5 (runner.py:150-151),
    at a non-square shape so a swapped index or stride cannot pass; C starts
    nonzero because the nest accumulates onto it."""
    M, K, N = 7, 13, 5
    A = np.fromfunction(lambda i, k: (i * K + k) % 7, (M, K), dtype=np.int64).astype(float)
    B = np.fromfunction(lambda k, j: (k * N + j) % 5, (K, N), dtype=np.int64).astype(float)
    C0 = np.arange(M * N, dtype=float).reshape(M, N) - 9.0
    a, b, c = _stride1000(A), _stride1000(B), _stride1000(C0)
    cref.matmul_f64_stride1000(a, b, c, M, K, N, variant=variant)
    got = np.array([[c[i * 1000 + j] for j in range(N)] for i in range(M)])
    want = C0 + np.array([[sum(A[i, t] * B[t, j] for t in range(K)) for j in range(N)]
                          for i in range(M)])
    assert np.array_equal(got, want)
    # cells between the rows' ends and the next row's start stay untouched
    assert not np.any(c[N:1000])
    with pytest.raises(ValueError):
        cref.matmul_f64_stride1000(a[:10], b, c, M, K, N)

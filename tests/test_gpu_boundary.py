"""The boundary's callers on the GPU: the benchmark verb, measured candidate
selection, workspaces under HIP graph capture, operands beyond 4 GiB, and
the reference's candidate loop with real launches (needs a gfx950 GPU).

Every launch goes through the C ABI; outputs are poisoned with INT32_MIN
first, and results are compared bit-exactly with the CPU oracle or checked
by exact properties where the oracle would take too long.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import gemm_oracle as go
from veritac_amd import _lib
from veritac_amd.specializations.hip_gemm import backend as hg
from veritac_amd.specializations.hip_gemm import runner
from veritac_amd.specializations.hip_gemm import verify

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


def rand_i8(dev, shape, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return torch.randint(-128, 128, shape, dtype=torch.int8, device=dev, generator=g)


# ---------------------------------------------------------------------------
# benchmark_gemm: the keys and protocol of cpu_gemm/runner.py:196-232
# ---------------------------------------------------------------------------

RUNNER_KEYS = {"gpu_time_ms", "cpu_time_ms", "speedup", "correct"}


@pytest.mark.parametrize("case", [
    dict(m=256, n=256, k=256, has_d=True, d_max_abs=1 << 20),
    dict(m=16, n=2048, k=1024),
    dict(m=1, n=4096, k=4096, variant="skinny_packed"),
    dict(m=512, n=1024, k=1024, batch=4, b_shared=True),
])
def test_benchmark_gemm_contract(dev, case):
    case = dict(case)
    variant = case.pop("variant", "auto")
    if variant == "auto":
        plan = hg.make_plan(**case)
    else:
        plan = dict(hg.make_plan(**case), variant=variant)
    say("benchmark_gemm", plan)
    res = runner.benchmark_gemm(plan, num_runs=5, warmup=2, cpu_budget_s=0.5)
    assert RUNNER_KEYS <= set(res)
    assert res["correct"] is True, res["check"]
    assert res["check"]["passed"] and res["check"]["cpu_rows_equal"]
    assert res["cpu_rows"] >= 1
    assert res["gpu_time_ms"] > 0 and res["cpu_time_ms"] > 0
    assert res["speedup"] == pytest.approx(res["cpu_time_ms"] / res["gpu_time_ms"])
    if variant == "skinny_packed":
        assert res["pack_ms"] is not None and res["pack_ms"] > 0


def test_benchmark_gemm_extrapolates_a_large_cpu_reference(dev):
    plan = hg.make_plan(2048, 2048, 2048)
    res = runner.benchmark_gemm(plan, num_runs=3, warmup=1, cpu_budget_s=0.05)
    assert res["correct"] is True
    assert res["cpu_extrapolated"] and res["cpu_rows"] < 2048
    assert res["speedup"] > 1


def test_benchmark_gemm_reports_a_wrong_result(dev, monkeypatch):
    """correct is False when the GPU output is wrong: a runner that drops
    the last K tile (a planted mistake on the GPU side of the comparison)."""
    plan = hg.make_plan(256, 256, 256)
    real = hg.native_runner

    def short_k(plan_, A, B, D, C, stream):
        cut = dict(plan_, k=plan_["k"] - 16)
        real(cut, A[:, :cut["k"]].contiguous(), B[:cut["k"]].contiguous(), D, C, stream)
        torch.cuda.synchronize()

    monkeypatch.setattr(hg, "native_runner", short_k)
    res = runner.benchmark_gemm(plan, num_runs=2, warmup=1, cpu_budget_s=0.05)
    assert res["correct"] is False


# ---------------------------------------------------------------------------
# optimize(measure=True): the measured selection of the candidates
# ---------------------------------------------------------------------------

def test_optimize_measure_picks_a_measured_correct_candidate(dev):
    r = hg.optimize(512, 512, 512, measure=True, num_runs=3)
    eligible = [c for c in r["candidates"] if c["valid"] and c["check"]["accepted"]]
    assert eligible and all(c["measured_ms"] and c["measured_correct"] for c in eligible)
    fastest = min(eligible, key=lambda c: c["measured_ms"])
    assert r["winner"] == fastest["plan"]
    for c in r["candidates"]:
        if not (c["valid"] and c["check"]["accepted"]):
            assert c["measured_ms"] is None


# ---------------------------------------------------------------------------
# The reference's candidate loop (examples/gemmini_gemm_demo.py:41-66) with
# real launches: every eligible candidate runs and equals the oracle.
# ---------------------------------------------------------------------------

def test_reference_candidate_loop_runs_every_eligible_plan(dev):
    m, n, k = 48, 64, 96   # not multiples of 16 in m: every variant's tails
    search = hg.optimize(m, n, k)
    rng = np.random.default_rng(7)
    A = rng.integers(-128, 128, (m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (k, n), dtype=np.int8)
    want = go.gemm_i8(A, B)
    ran = 0
    for entry in search["candidates"]:
        if not entry["valid"] or not entry["check"]["accepted"]:
            continue
        C = torch.full((m, n), INT32_MIN, dtype=torch.int32, device=dev)
        hg.run(entry["plan"], torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev), out=C)
        torch.cuda.synchronize()
        assert np.array_equal(C.cpu().numpy(), want), entry["plan"]["variant"]
        ran += 1
    assert ran >= 4 and search["winner"] is not None


# ---------------------------------------------------------------------------
# Workspaces and HIP graph capture
# ---------------------------------------------------------------------------

def _decode(dev, n, k, seed):
    A = rand_i8(dev, (16, k), seed)
    B = rand_i8(dev, (k, n), seed + 1)
    return A, B


def _ws_bytes(plan):
    st, reason, _, _, ws = _lib.gemm_check(plan["m"], plan["n"], plan["k"], plan["k"], plan["n"],
                                            plan["n"], plan["n"], variant=plan["variant"],
                                            k_split=plan["k_split"])
    assert st == 0, reason
    return ws


def test_graph_replay_survives_workspace_growth(dev):
    """A K-split decode captured into a graph keeps working after a larger
    call on the same stream grows the workspace: the superseded workspace is
    never freed. Every replay, with eager work and synchronization between
    replays, equals the eager result and the oracle."""
    small = hg.make_plan(16, 2048, 4096)
    big = hg.make_plan(16, 14336, 4096, k_split=8)
    assert small["variant"] == big["variant"] == "skinny"
    assert _ws_bytes(small) > 0 and _ws_bytes(big) > 2 * _ws_bytes(small)
    s = torch.cuda.Stream(device=dev)
    A, B = _decode(dev, 2048, 4096, 11)
    A2, B2 = _decode(dev, 14336, 4096, 13)
    C = torch.empty((16, 2048), dtype=torch.int32, device=dev)
    C2 = torch.empty((16, 14336), dtype=torch.int32, device=dev)
    want = go.gemm_i8(A.cpu().numpy(), B.cpu().numpy())
    want2 = go.gemm_i8(A2.cpu().numpy(), B2.cpu().numpy())
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        hg.run(small, A, B, out=C, stream=s.cuda_stream)      # the stream's first workspace
    s.synchronize()
    assert np.array_equal(C.cpu().numpy(), want)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        hg.run(small, A, B, out=C, stream=s.cuda_stream)
    for i in range(4):
        C.fill_(INT32_MIN)
        C2.fill_(INT32_MIN)
        with torch.cuda.stream(s):
            if i == 1:
                # grows the stream's workspace past the captured one
                hg.run(big, A2, B2, out=C2, stream=s.cuda_stream)
            g.replay()
        s.synchronize()
        say("replay", i)
        assert np.array_equal(C.cpu().numpy(), want), "replay %d" % i
        if i == 1:
            assert np.array_equal(C2.cpu().numpy(), want2)


def test_workspace_growth_during_capture_is_refused(dev):
    """A call that needs workspace its stream does not have yet is refused
    while the stream is being captured (nothing is allocated in capture)."""
    plan = hg.make_plan(16, 4096, 8192, k_split=16)
    assert plan["variant"] == "skinny" and _ws_bytes(plan) > 0
    s = torch.cuda.Stream(device=dev)      # fresh stream: no workspace
    A, B = _decode(dev, 4096, 8192, 17)
    C = torch.empty((16, 4096), dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(hg.HipGemmError) as exc:
        with torch.cuda.graph(g, stream=s):
            hg.run(plan, A, B, out=C, stream=s.cuda_stream)
    assert "before capture" in str(exc.value)
    assert exc.value.code == _lib.VT_EUNSUPPORTED
    torch.cuda.synchronize()
    # after an eager call the same capture succeeds and replays correctly
    with torch.cuda.stream(s):
        hg.run(plan, A, B, out=C, stream=s.cuda_stream)
    s.synchronize()
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=s):
        hg.run(plan, A, B, out=C, stream=s.cuda_stream)
    want = go.gemm_i8(A.cpu().numpy(), B.cpu().numpy())
    for i in range(3):
        C.fill_(INT32_MIN)
        with torch.cuda.stream(s):
            g2.replay()
        s.synchronize()
        assert np.array_equal(C.cpu().numpy(), want), "replay %d" % i


# ---------------------------------------------------------------------------
# Operands beyond 4 GiB through the MFMA variants (64-bit tile bases)
# ---------------------------------------------------------------------------

def _check_big(A, B, C, rows_to_compare):
    """Full output by exact projections over row blocks, and chosen rows
    element by element against the oracle."""
    step = 1 << 17
    for r0 in range(0, A.shape[0], step):
        r1 = min(A.shape[0], r0 + step)
        res = verify.exact_check(A[r0:r1], B, C[r0:r1], vectors=8, seed=r0)
        assert res["passed"], (r0, res)
    Bn = B.cpu().numpy()
    for r in rows_to_compare:
        got = C[r].cpu().numpy()
        want = go.gemm_i8(A[r:r + 1].cpu().numpy(), Bn)[0]
        assert np.array_equal(got, want), "row %d" % r


@pytest.mark.parametrize("variant,m", [("mfma_256x256", (1 << 20) + 256),
                                       ("mfma_256x128", (1 << 20) + 256),
                                       ("mfma_128x128", (1 << 20) + 200)])
def test_mfma_variants_address_a_beyond_4gib(dev, variant, m):
    k, n = 4096, 256
    assert m * k > 2**32
    say("A beyond 4 GiB:", variant, m, n, k)
    A = rand_i8(dev, (m, k), 23)
    B = rand_i8(dev, (k, n), 29)
    C = torch.full((m, n), INT32_MIN, dtype=torch.int32, device=dev)
    plan = dict(hg.make_plan(m, n, k), variant=variant)
    hg.run(plan, A, B, out=C)
    torch.cuda.synchronize()
    edge = 2**32 // k            # first row whose offset from A passes 2^32
    rows = [0, 1, edge - 1, edge, edge + 1, m - 2, m - 1]
    _check_big(A, B, C, rows)
    del A, C
    torch.cuda.empty_cache()



# ---------------------------------------------------------------------------
# Decode K splits: the slices' partial sums and the reduction kernel
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("m,n,k,k_split,with_d,batch", [
    (1, 14336, 4096, 0, False, 1), (2, 14336, 4096, 0, True, 1), (1, 4112, 2048, 3, True, 1),
    (2, 1024, 8192, 16, False, 1), (1, 272, 4096, 64, True, 2), (2, 2048, 1024, 7, True, 3)])
def test_k_split_decode_in_place(dev, m, n, k, k_split, with_d, batch):
    """C = D + A.B through the skinny kernel with K split across workgroups
    (in place: C is D), for ragged N, batches and split counts from 3 to 64."""
    rng = np.random.default_rng(m * 1000 + n + k_split)
    A = rng.integers(-128, 128, (batch, m, k), dtype=np.int8)
    B = rng.integers(-128, 128, (batch, k, n), dtype=np.int8)
    D = rng.integers(-2**20, 2**20, (batch, m, n), dtype=np.int32) if with_d else None
    plan = hg.make_plan(m, n, k, batch=batch, has_d=with_d, d_max_abs=(1 << 20) if with_d else 0,
                        variant="skinny", k_split=k_split)
    assert hg.skinny_split(plan)[0] > 1
    # the plan's operand shapes: 2-D for one batch, 3-D (B per batch) otherwise
    lead = (lambda x: x[0]) if batch == 1 else (lambda x: x)
    At = torch.from_numpy(lead(A)).to(dev)
    Bt = torch.from_numpy(lead(B)).to(dev)
    if with_d:
        C = torch.from_numpy(np.ascontiguousarray(lead(D))).to(dev)
        out = hg.run(plan, At, Bt, C, out=C)
    else:
        out = hg.run(plan, At, Bt, out=torch.full(lead(np.zeros((batch, m, n))).shape, INT32_MIN,
                                                    dtype=torch.int32, device=dev))
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(batch, m, n)
    for b in range(batch):
        assert np.array_equal(got[b], go.gemm_i8(A[b], B[b], None if D is None else D[b])), b


def test_k_split_workspace_shared_by_calls_and_replays(dev):
    """Two decode calls (different N and K split) share the stream's
    partial-sum workspace: captured in one graph and replayed with an eager
    call on the same stream between replays, every replay checked."""
    s = torch.cuda.Stream(device=dev)
    cases = []
    for m, n, k, ks in ((1, 14336, 4096, 4), (2, 3072, 4096, 9)):
        A, B = rand_i8(dev, (m, k), m + n), rand_i8(dev, (k, n), k + n)
        plan = hg.make_plan(m, n, k, variant="skinny", k_split=ks)
        C = torch.empty((m, n), dtype=torch.int32, device=dev)
        cases.append((plan, A, B, C, go.gemm_i8(A.cpu().numpy(), B.cpu().numpy())))
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        for plan, A, B, C, _ in cases:
            hg.run(plan, A, B, out=C, stream=s.cuda_stream)
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for plan, A, B, C, _ in cases:
            hg.run(plan, A, B, out=C, stream=s.cuda_stream)
    for i in range(4):
        for _, _, _, C, _ in cases:
            C.fill_(INT32_MIN)
        with torch.cuda.stream(s):
            g.replay()
            # an eager call between replays on the same stream and workspace
            plan, A, B, C, _ = cases[i % 2]
            hg.run(plan, A, B, out=C, stream=s.cuda_stream)
            g.replay()
        s.synchronize()
        for plan, A, B, C, want in cases:
            assert np.array_equal(C.cpu().numpy(), want), (i, plan["n"])

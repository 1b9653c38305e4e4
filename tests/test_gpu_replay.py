"""GPU command-stream replay (vt_replay_i8 via specializations/hip_gemm/
replay.py) against the recorded Spike outputs, the oracle interpreter and
vt_gemm_i8 (needs a gfx950 GPU)."""
import copy

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from conftest import decode_cout, witness_inputs
from oracle import gemm_oracle as go
from oracle import gemmini_replay as gr
from veritac_amd import _lib
from veritac_amd.specializations.hip_gemm import replay as rp

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    assert _lib.load_library().vt_device_count() >= 1, "GPU visible but not gfx950"
    return torch.device("cuda", 0)


def say(*args):
    print(*args, flush=True)


def spike_inputs(plan, mode):
    a, b = go.fill_inputs(mode, plan["m"] * plan["k"], plan["k"] * plan["n"])
    return [go.to_int8(x) for x in a], [go.to_int8(x) for x in b]


def hip_gemm(dev, A, B, p):
    At = torch.tensor(A, dtype=torch.int8, device=dev)
    Bt = torch.tensor(B, dtype=torch.int8, device=dev)
    C = torch.empty(p["m"] * p["n"], dtype=torch.int32, device=dev)
    m, n, k = p["m"], p["n"], p["k"]
    _lib.gemm_raw(At.data_ptr(), Bt.data_ptr(), None, C.data_ptr(), m, n, k, k, n, n, n)
    _lib.sync(None)
    return C.cpu().tolist()


def test_replay_reproduces_the_recorded_spike_outputs(dev, commands, golden):
    runs = {r["name"]: r for r in golden["runs"]}
    for s in (x for x in commands if "spike_run" in x):
        for mode in go.SPIKE_MODES:
            say("replay", s["name"], mode)
            A, B = spike_inputs(s["plan"], mode)
            C, stats = rp.run_commands(s["commands"], s["plan"], A, B, device=dev)
            assert C == decode_cout(runs[s["spike_run"]]["cout"][mode]), (s["name"], mode)


def test_replay_equals_oracle_and_hip_gemm_on_every_certified_stream(dev, commands):
    rng = np.random.default_rng(7)
    for s in commands:
        if "witness" in s:
            continue
        p = s["plan"]
        say("replay vs gemm", s["name"])
        for trial in range(2):
            A = rng.integers(-128, 128, p["m"] * p["k"]).tolist()
            B = rng.integers(-128, 128, p["k"] * p["n"]).tolist()
            C, stats = rp.run_commands(s["commands"], p, A, B, device=dev)
            want, want_stats = gr.run_commands(s["commands"], p, A, B)
            assert C == want and stats == want_stats, s["name"]
            assert C == hip_gemm(dev, A, B, p), s["name"]


def test_replay_reproduces_each_rejection_witness(dev, commands):
    for s in (x for x in commands if "witness" in x):
        say("witness", s["name"])
        w, p = s["witness"], s["plan"]
        A, B = witness_inputs(s)
        C, _ = rp.run_commands(s["commands"], p, A, B, device=dev)
        assert C == gr.run_commands(s["commands"], p, A, B)[0]
        assert C[w["row"] * p["n"] + w["col"]] == w["actual"]
        assert hip_gemm(dev, A, B, p)[w["row"] * p["n"] + w["col"]] == w["expected"]


def test_replay_extremes_stay_exact(dev, commands):
    s = next(x for x in commands if x["name"] == "checked_general/64x64x64_reuse_b")
    p = s["plan"]
    for a, b in ((-128, -128), (127, -128)):
        A = [a] * (p["m"] * p["k"])
        B = [b] * (p["k"] * p["n"])
        C, _ = rp.run_commands(s["commands"], p, A, B, device=dev)
        assert C == [a * b * p["k"]] * (p["m"] * p["n"])


def test_replay_reports_int32_overflow_like_the_oracle(dev, commands):
    s = copy.deepcopy(next(x for x in commands if x["name"] == "checked/16x16x16_baseline"))
    cmds, p = s["commands"], s["plan"]
    i = max(j for j, c in enumerate(cmds) if c["kind"] == "compute")
    pre = dict(next(c for c in cmds if c["kind"] == "preload"), bd_spad_addr=rp.GARBAGE_ADDR)
    pre["out_addr"] |= rp.ACCUMULATE_BIT
    comp = dict(cmds[i], accumulated=True)
    cmds = cmds[:i + 1] + [pre, comp] * 8200 + cmds[i + 1:]
    A = [-128] * 256
    B = [-128] * 256
    with pytest.raises(gr.ReplayError):
        gr.run_commands(cmds, p, A, B)
    with pytest.raises(_lib.HipGemmError, match="overflow"):
        rp.run_commands(cmds, p, A, B, device=dev)
    # 8190 accumulates stay below 2^31: same result as the oracle
    cmds_ok = s["commands"][:i + 1] + [pre, comp] * 8190 + s["commands"][i + 1:]
    C, _ = rp.run_commands(cmds_ok, p, A, B, device=dev)
    assert C == gr.run_commands(cmds_ok, p, A, B)[0] == [16384 * 16 * 8191] * 256


def test_replay_repeated_calls_are_independent(dev, commands):
    s = next(x for x in commands if x["name"] == "checked_general/32x16x32_reuse_b")
    p = s["plan"]
    rng = np.random.default_rng(3)
    for it in range(5):
        A = rng.integers(-128, 128, p["m"] * p["k"]).tolist()
        B = rng.integers(-128, 128, p["k"] * p["n"]).tolist()
        assert rp.run_commands(s["commands"], p, A, B, device=dev)[0] == \
            gr.run_commands(s["commands"], p, A, B)[0]

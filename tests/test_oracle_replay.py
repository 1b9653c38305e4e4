"""Pins of the command-stream oracle (oracle/gemmini_replay.py), CPU only.

The replay of the reference's own command streams must reproduce the Spike
outputs it recorded, every certified stream must compute A.B, each rejection
witness must reproduce its recorded wrong cell, and planted faults must raise.
"""
import copy

import numpy as np
import pytest

from conftest import decode_cout, witness_inputs
from oracle import gemm_oracle as go
from oracle import gemmini_replay as gr


def spike_inputs(plan, mode):
    a, b = go.fill_inputs(mode, plan["m"] * plan["k"], plan["k"] * plan["n"])
    return [go.to_int8(x) for x in a], [go.to_int8(x) for x in b]


def test_linked_streams_reproduce_the_recorded_spike_outputs(commands, golden):
    runs = {r["name"]: r for r in golden["runs"]}
    linked = [s for s in commands if "spike_run" in s]
    assert len(linked) == 8
    for s in linked:
        for mode in go.SPIKE_MODES:
            A, B = spike_inputs(s["plan"], mode)
            C, stats = gr.run_commands(s["commands"], s["plan"], A, B)
            assert C == decode_cout(runs[s["spike_run"]]["cout"][mode]), (s["name"], mode)
            p = s["plan"]
            assert stats["macs"] == p["m"] * p["n"] * p["k"]


def test_certified_streams_compute_the_gemm(commands):
    rng = np.random.default_rng(0)
    for s in commands:
        if "witness" in s:
            continue
        p = s["plan"]
        A = rng.integers(-128, 128, p["m"] * p["k"]).tolist()
        B = rng.integers(-128, 128, p["k"] * p["n"]).tolist()
        C, _ = gr.run_commands(s["commands"], p, A, B)
        want = go.gemm_i8(np.array(A, np.int8).reshape(p["m"], p["k"]),
                          np.array(B, np.int8).reshape(p["k"], p["n"]))
        assert C == want.reshape(-1).tolist(), s["name"]


def test_rejection_witnesses_reproduce_their_wrong_cell(commands):
    witnesses = [s for s in commands if "witness" in s]
    assert len(witnesses) == 4
    for s in witnesses:
        w, p = s["witness"], s["plan"]
        A, B = witness_inputs(s)
        C, _ = gr.run_commands(s["commands"], p, A, B)
        want = go.gemm_i8(np.array(A, np.int8).reshape(p["m"], p["k"]),
                          np.array(B, np.int8).reshape(p["k"], p["n"]))
        assert C[w["row"] * p["n"] + w["col"]] == w["actual"]
        assert want[w["row"], w["col"]] == w["expected"] != w["actual"]


def _stream(commands, name):
    return next(s for s in commands if s["name"] == name)


def test_hand_known_answer_16cube():
    """A = 2*I (16x16), B[t][j] = t - j: C = 2*B, by hand."""
    plan = {"m": 16, "n": 16, "k": 16, "dim": 16, "schedule": "baseline",
            "scratchpad_rows": 32, "accumulator_rows": 16}
    A = [2 if i == t else 0 for i in range(16) for t in range(16)]
    B = [t - j for t in range(16) for j in range(16)]
    cmds = [{"kind": "config_ex", "dataflow": 1}, {"kind": "config_st", "stride_bytes": 64},
            {"kind": "config_ld", "slot": 0, "stride_bytes": 16, "scale": 1.0},
            {"kind": "config_ld", "slot": 1, "stride_bytes": 16, "scale": 1.0},
            {"kind": "mvin", "slot": 0, "buf": "A", "offset": 0, "spad_addr": 0, "cols": 16, "rows": 16},
            {"kind": "mvin", "slot": 1, "buf": "B", "offset": 0, "spad_addr": 16, "cols": 16, "rows": 16},
            {"kind": "preload", "bd_spad_addr": 16, "out_addr": gr.ACC_SPACE_BIT | gr.FULL_C_BIT},
            {"kind": "compute", "accumulated": False, "a_spad_addr": 0, "bd_spad_addr": gr.GARBAGE_ADDR},
            {"kind": "mvout", "buf_offset": 0, "acc_addr": gr.ACC_SPACE_BIT | gr.FULL_C_BIT, "cols": 16, "rows": 16},
            {"kind": "fence"}]
    C, stats = gr.run_commands(cmds, plan, A, B)
    assert C == [2 * (t - j) for t in range(16) for j in range(16)]
    assert stats == {"instructions": 10, "macs": 4096, "overwrites": 16, "accumulates": 0}


@pytest.mark.parametrize("fault", ["drop_fence", "fresh_accumulate", "drop_mvout", "overflow",
                                   "bad_acc_space", "b_not_moved_in", "accumulated_without_b"])
def test_planted_faults_raise(commands, fault):
    s = copy.deepcopy(_stream(commands, "checked_general/32x16x32_baseline"))
    cmds, p = s["commands"], s["plan"]
    A = [1] * (p["m"] * p["k"])
    B = [1] * (p["k"] * p["n"])
    if fault == "drop_fence":
        cmds = [c for c in cmds if c["kind"] != "fence"]
    elif fault == "fresh_accumulate":
        pre = next(c for c in cmds if c["kind"] == "preload")
        pre["out_addr"] |= gr.ACCUMULATE_BIT
    elif fault == "drop_mvout":
        i = max(i for i, c in enumerate(cmds) if c["kind"] == "mvout")
        cmds = cmds[:i] + cmds[i + 1:]
    elif fault == "overflow":
        p = dict(p, k=32)
        A = [-128] * (p["m"] * p["k"])
        B = [-128] * (p["k"] * p["n"])
        # 32 * 16384 = 524288 fits; accumulate the same tile 5000 times instead
        comp = [c for c in cmds if c["kind"] in ("preload", "compute")][-2:]
        acc_pre = dict(comp[0], out_addr=comp[0]["out_addr"] | gr.ACCUMULATE_BIT, bd_spad_addr=gr.GARBAGE_ADDR)
        acc_cmp = dict(comp[1], accumulated=True)
        i = max(i for i, c in enumerate(cmds) if c["kind"] == "compute")
        cmds = cmds[:i + 1] + [acc_pre, acc_cmp] * 8200 + cmds[i + 1:]
    elif fault == "bad_acc_space":
        mv = next(c for c in cmds if c["kind"] == "mvout")
        mv["acc_addr"] &= ~gr.ACC_SPACE_BIT
    elif fault == "b_not_moved_in":
        p = dict(p, scratchpad_rows=64)
        next(c for c in cmds if c["kind"] == "preload")["bd_spad_addr"] = 48
    elif fault == "accumulated_without_b":
        comp = next(c for c in cmds if c["kind"] == "compute")
        comp["accumulated"] = True
    with pytest.raises(gr.ReplayError):
        gr.run_commands(cmds, p, A, B)
    s_ok = _stream(commands, "checked_general/32x16x32_baseline")
    gr.run_commands(s_ok["commands"], s_ok["plan"], [1] * 1024, [1] * 512)


def test_plan_validation_boundaries():
    plan = {"m": 16, "n": 16, "k": 131056, "dim": 16, "schedule": "baseline",
            "scratchpad_rows": 32, "accumulator_rows": 16}
    assert gr.validate_plan(plan)[0]
    assert not gr.validate_plan(dict(plan, k=131072))[0]
    assert not gr.validate_plan(dict(plan, accumulator_rows=15))[0]
    assert not gr.validate_plan(dict(plan, scratchpad_rows=31))[0]
    assert not gr.validate_plan(dict(plan, schedule="reuse_b", m=32, accumulator_rows=31))[0]
    assert gr.validate_plan(dict(plan, schedule="reuse_b", m=32, accumulator_rows=32))[0]
    assert not gr.validate_plan(dict(plan, m=True))[0]

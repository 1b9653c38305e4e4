"""Host side of the GPU command-stream replay (no GPU needed): the static
lowering accepts exactly the streams the oracle interpreter accepts, reports
the same statistics, and emits a tile program whose content is checked
against the commands."""
import copy

import numpy as np
import pytest

from oracle import gemmini_replay as gr
from veritac_amd import _lib
from veritac_amd.specializations.hip_gemm import replay as rp


def test_constants_match_the_oracle():
    for name in ("DIM", "GARBAGE_ADDR", "ACC_SPACE_BIT", "ACCUMULATE_BIT", "FULL_C_BIT",
                 "SCRATCHPAD_ROWS", "ACC_ROWS", "WEIGHT_STATIONARY"):
        assert getattr(rp, name) == getattr(gr, name), name


def test_every_fixture_stream_lowers_with_the_oracle_statistics(commands):
    rng = np.random.default_rng(1)
    for s in commands:
        p = s["plan"]
        program, stats = rp.lower(s["commands"], p)
        A = rng.integers(-3, 4, p["m"] * p["k"]).tolist()
        B = rng.integers(-3, 4, p["k"] * p["n"]).tolist()
        _, want = gr.run_commands(s["commands"], p, A, B)
        assert stats == want, s["name"]
        kinds = [c["kind"] for c in s["commands"]]
        assert (program[:, 0] == _lib.REPLAY_MVIN).sum() == kinds.count("mvin")
        assert (program[:, 0] == _lib.REPLAY_COMPUTE).sum() == kinds.count("compute")
        assert (program[:, 0] == _lib.REPLAY_MVOUT).sum() == kinds.count("mvout")
        preloaded = sum(1 for c in s["commands"] if c["kind"] == "compute" and not c["accumulated"])
        assert (program[:, 0] == _lib.REPLAY_LATCH_B).sum() == preloaded
        assert list(program[:, 7]) == sorted(program[:, 7])      # stream order kept


def test_program_words_follow_the_commands(commands):
    s = next(x for x in commands if x["name"] == "checked/16x16x16_baseline")
    program, _ = rp.lower(s["commands"], s["plan"])
    assert program.tolist() == [
        [_lib.REPLAY_MVIN, 0, 0, 16, 0, 0, 0, 4],
        [_lib.REPLAY_MVIN, 1, 0, 16, 16, 0, 0, 5],
        [_lib.REPLAY_LATCH_B, 16, 0, 0, 0, 0, 0, 7],
        [_lib.REPLAY_COMPUTE, 0, 0, 0, 0, 0, 0, 7],
        [_lib.REPLAY_MVOUT, 0, 0, 16, 0, 0, 0, 8]]


MUTATIONS = {
    "drop_fence": lambda c: [x for x in c if x["kind"] != "fence"],
    "drop_last_mvout": lambda c: c[:max(i for i, x in enumerate(c) if x["kind"] == "mvout")]
    + c[max(i for i, x in enumerate(c) if x["kind"] == "mvout") + 1:],
    "drop_config_ex": lambda c: [x for x in c if x["kind"] != "config_ex"],
    "drop_config_st": lambda c: [x for x in c if x["kind"] != "config_st"],
    "drop_first_mvin": lambda c: c[:min(i for i, x in enumerate(c) if x["kind"] == "mvin")]
    + c[min(i for i, x in enumerate(c) if x["kind"] == "mvin") + 1:],
}


def _mutate(cmds, what):
    cmds = copy.deepcopy(cmds)
    if what in MUTATIONS:
        return MUTATIONS[what](cmds)
    first = lambda kind: next(x for x in cmds if x["kind"] == kind)
    if what == "accumulate_first":
        first("preload")["out_addr"] |= rp.ACCUMULATE_BIT
    elif what == "overwrite_later":     # turns a k>0 accumulate into an overwrite: valid, wrong C
        pre = [x for x in cmds if x["kind"] == "preload" and x["out_addr"] & rp.ACCUMULATE_BIT]
        if not pre:
            return None
        pre[0]["out_addr"] &= ~rp.ACCUMULATE_BIT
    elif what == "scratch_acc_bit":
        first("mvout")["acc_addr"] &= ~rp.ACC_SPACE_BIT
    elif what == "narrow_c":
        first("mvout")["acc_addr"] &= ~rp.FULL_C_BIT
    elif what == "partial_tile":
        first("mvin")["rows"] = 8
    elif what == "bad_dataflow":
        first("config_ex")["dataflow"] = 0
    elif what == "scale":
        first("config_ld")["scale"] = 0.5
    elif what == "bd_not_garbage":
        first("compute")["bd_spad_addr"] = 0
    elif what == "accumulated_first":
        first("compute")["accumulated"] = True
    elif what == "out_of_range_mvin":
        first("mvin")["offset"] = 10**7
    elif what == "acc_beyond":
        first("preload")["out_addr"] = rp.ACC_SPACE_BIT | rp.FULL_C_BIT | 4000
    elif what == "unknown_kind":
        cmds.insert(1, {"kind": "flush"})
    elif what == "short_store_stride":
        first("config_st")["stride_bytes"] = 4
    return cmds


@pytest.mark.parametrize("what", list(MUTATIONS) + [
    "accumulate_first", "overwrite_later", "scratch_acc_bit", "narrow_c", "partial_tile",
    "bad_dataflow", "scale", "bd_not_garbage", "accumulated_first", "out_of_range_mvin",
    "acc_beyond", "unknown_kind", "short_store_stride"])
def test_lowering_accepts_exactly_what_the_oracle_accepts(commands, what):
    checked = 0
    for s in commands:
        cmds = _mutate(s["commands"], what)
        if cmds is None:
            continue
        p = s["plan"]
        A = [1] * (p["m"] * p["k"])
        B = [1] * (p["k"] * p["n"])
        try:
            gr.run_commands(cmds, p, A, B)
            oracle_ok = True
        except gr.ReplayError:
            oracle_ok = False
        try:
            rp.lower(cmds, p)
            host_ok = True
        except _lib.HipGemmError:
            host_ok = False
        assert host_ok == oracle_ok, (s["name"], what)
        checked += 1
    assert checked > 0


def test_plan_validation_matches_the_oracle():
    base = {"m": 32, "n": 16, "k": 32, "dim": 16, "schedule": "reuse_b",
            "scratchpad_rows": 32, "accumulator_rows": 32}
    for change in ({}, {"k": 131072}, {"k": 131056}, {"accumulator_rows": 31},
                   {"scratchpad_rows": 31}, {"scratchpad_rows": 16385}, {"dim": 8},
                   {"schedule": "os"}, {"m": 24}, {"m": True}, {"accumulator_rows": 1025}):
        plan = dict(base, **change)
        assert rp.validate_plan(plan)[0] == gr.validate_plan(plan)[0], change


def test_run_commands_refuses_bad_inputs_before_the_device(commands):
    s = commands[0]
    p = s["plan"]
    with pytest.raises(_lib.HipGemmError):
        rp.run_commands(s["commands"], p, [0] * 5, [0] * (p["k"] * p["n"]))
    with pytest.raises(_lib.HipGemmError):
        rp.run_commands(s["commands"], p, [300] * (p["m"] * p["k"]), [0] * (p["k"] * p["n"]))
    with pytest.raises(_lib.HipGemmError):
        rp.run_commands(s["commands"], p, [0] * (p["m"] * p["k"]), [0] * (p["k"] * p["n"]),
                        device="cpu")

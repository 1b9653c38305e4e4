"""Gemmini schedule generators, modeled counts and the symbolic program check
(no GPU needed).

The generators are pinned command for command by the streams the reference
recorded from its own generators (benchmarks/gemmini/checked/*,
checked_general/* and the ai_repair edge, in tests/golden/
gemmini_commands.json). The program check is pinned by the reference's
recorded verdicts: every certified stream accepted, the four blind-search
rejection witnesses refused at their recorded cell. The remaining cases
restate tests/test_gemmini.py:77-93 and tests/test_gemmini_general.py of the
reference, and a mutation sweep ties acceptance to the oracle interpreter:
every stream the check accepts computes the GEMM.
"""
import copy
import random

import pytest

from oracle import gemm_oracle as go
from oracle import gemmini_replay as gr
from veritac_amd.specializations.hip_gemm import schedules as sc

UNSEEN = ((32, 16, 32), (16, 32, 48), (48, 32, 64), (64, 64, 64))
MODES = ("zero", "max", "min", "minmax", "lcg")


def oracle_equals_gemm(plan, cmds, seed=917, modes=MODES):
    m, n, k = plan["m"], plan["n"], plan["k"]
    for mode in modes:
        A, B = go.deterministic_inputs(m, n, k, seed, mode)
        C, stats = gr.run_commands(cmds, plan, A, B)
        if C != go.scalar_matmul(A, B, m, n, k):
            return False
        assert stats["macs"] == m * n * k
    return True


def test_generators_reproduce_every_recorded_generated_stream(commands):
    seen = 0
    for s in commands:
        if s["name"].startswith(("checked/", "checked_general/")):
            assert sc.gen_commands(s["plan"]) == s["commands"], s["name"]
            seen += 1
    assert seen == 9


def test_the_ai_repair_edge_is_baseline_to_batched_reuse(commands):
    """The accepted rewrite edge of benchmarks/gemmini/ai_repair: its source
    is the baseline stream. Its destination walks the tiles of
    gen_batched_reuse_b(plan, 2) -- the same moves, addresses and outputs in
    the same order -- but latches B by an explicit preload on every compute,
    where lowering.py:33-34 retains it after a batch's first compute."""
    by = {s["name"]: s for s in commands}
    src = by["ai_repair/2026-09-16/accepted_edge/source"]
    dst = by["ai_repair/2026-09-16/accepted_edge/destination"]
    assert src["plan"] == dst["plan"]
    assert sc.gen_baseline(src["plan"]) == src["commands"]
    gen = sc.gen_batched_reuse_b(dst["plan"], 2)
    assert sum(c["kind"] == "compute" and c["accumulated"] for c in gen) == 2
    relatched = copy.deepcopy(gen)
    for c in relatched:
        if c["kind"] == "preload":
            c["bd_spad_addr"] = sc.B_SPAD
        elif c["kind"] == "compute":
            c["accumulated"] = False
    assert relatched == dst["commands"]
    for cmds in (gen, relatched):
        assert sc.check_program(dst["plan"], cmds)[:2] == (True, "accepted")


def test_reuse_b_is_one_batch_of_every_row():
    for m, n, k in UNSEEN:
        plan = sc.make_plan(m, n, k, "reuse_b")
        assert sc.gen_reuse_b(plan) == sc.gen_batched_reuse_b(plan, m // 16)


def test_make_plan_capacities():
    """tests/test_gemmini.py:25-47 of the reference."""
    plan = sc.make_plan(32, 32, 32, "baseline")
    assert (plan["dim"], plan["scratchpad_rows"], plan["accumulator_rows"]) == (16, 32, 16)
    plan = sc.make_plan(48, 32, 64, "reuse_b")
    assert (plan["scratchpad_rows"], plan["accumulator_rows"]) == (32, 48)
    for schedule in sc.SCHEDULES:
        for shape in ((16, 16, 16), (32, 32, 32), (48, 32, 64)):
            assert gr.validate_plan(sc.make_plan(*shape, schedule))[0]


def test_command_structure_counts():
    """tests/test_gemmini.py:77-93 of the reference."""
    base = sc.modeled_counts(sc.gen_commands(sc.make_plan(32, 32, 32, "baseline")))
    assert (base["mvin_A"], base["mvin_B"], base["mvout"], base["fence"]) == (8, 8, 4, 1)
    reuse = sc.modeled_counts(sc.gen_commands(sc.make_plan(32, 32, 32, "reuse_b")))
    assert (reuse["mvin_A"], reuse["mvin_B"], reuse["mvout"], reuse["fence"]) == (8, 4, 4, 1)
    assert reuse["mvin_B"] < base["mvin_B"] and reuse["dma_bytes"] < base["dma_bytes"]


def test_counts_follow_the_stream_and_closed_forms():
    for m, n, k in UNSEEN + ((80, 48, 32),):
        it, jt, kt = m // 16, n // 16, k // 16
        for schedule, b_tiles in (("baseline", it * jt * kt), ("reuse_b", jt * kt)):
            cmds = sc.gen_commands(sc.make_plan(m, n, k, schedule))
            c = sc.modeled_counts(cmds)
            assert c["mvin_A"] == it * jt * kt and c["mvin_B"] == b_tiles
            assert c["compute"] == c["preload"] == it * jt * kt
            assert c["compute_preloaded"] == (it * jt * kt if schedule == "baseline" else jt * kt)
            assert c["mvout"] == it * jt and c["instructions"] == len(cmds)
            assert c["dma_bytes"] == 256 * (c["mvin_A"] + c["mvin_B"]) + 1024 * c["mvout"]
            assert sc.modeled_objective(c) == (c["dma_bytes"], len(cmds))
        for batch in (1, 2, 3):
            c = sc.modeled_counts(sc.gen_batched_reuse_b(sc.make_plan(m, n, k, "reuse_b"), batch))
            assert c["mvin_B"] == jt * kt * -(-it // batch)


def test_optimize_selects_reuse_b_unless_the_accumulator_is_too_small():
    r = sc.optimize(32, 32, 32)
    assert r["winner"]["schedule"] == "reuse_b"
    assert all(c["check"]["accepted"] for c in r["candidates"])
    r = sc.optimize(64, 16, 16, accumulator_rows=32)
    by = {c["plan"]["schedule"]: c for c in r["candidates"]}
    assert not by["reuse_b"]["valid"] and "accumulator_rows" in by["reuse_b"]["invalid_reason"]
    assert r["winner"]["schedule"] == "baseline"
    assert sc.optimize(16, 16, 24)["winner"] is None


def test_check_accepts_every_certified_stream_and_refuses_each_witness(commands):
    for s in commands:
        ok, why, _ = sc.check_program(s["plan"], s["commands"])
        if "witness" in s:
            w = s["witness"]
            assert not ok and why.startswith(sc.OUTPUT_MISMATCH), s["name"]
            assert "row %d, col %d" % (w["row"], w["col"]) in why, (s["name"], why)
        else:
            assert ok, (s["name"], why)


def test_unseen_shapes_both_schedules():
    """tests/test_gemmini_general.py:13-19 of the reference, and the oracle
    interpreter's result equals the GEMM."""
    for shape in UNSEEN:
        for schedule in sc.SCHEDULES:
            plan = sc.make_plan(*shape, schedule)
            cmds = sc.gen_commands(plan)
            assert sc.check_program(plan, cmds)[:2] == (True, "accepted"), (shape, schedule)
            assert oracle_equals_gemm(plan, cmds, modes=("lcg", "minmax"))


def test_independent_output_tiles_can_be_reversed():
    """tests/test_gemmini_general.py:21-28."""
    plan = sc.make_plan(32, 16, 32, "baseline")
    cmds = sc.gen_commands(plan)
    rev = cmds[:4] + cmds[13:22] + cmds[4:13] + cmds[-1:]
    assert rev != cmds
    assert sc.check_program(plan, rev)[:2] == (True, "accepted")
    assert oracle_equals_gemm(plan, rev, modes=("lcg",))


def test_partial_sum_overwrite_is_rejected():
    """tests/test_gemmini_general.py:30-35: the interpreter runs the stream
    (a wrong C); the check refuses it."""
    plan = sc.make_plan(32, 16, 32, "baseline")
    cmds = copy.deepcopy(sc.gen_commands(plan))
    next(c for c in cmds if c["kind"] == "preload" and c["out_addr"] & sc.ACCUMULATE_BIT)[
        "out_addr"] &= ~sc.ACCUMULATE_BIT
    ok, why, _ = sc.check_program(plan, cmds)
    assert not ok and why.startswith(sc.OUTPUT_MISMATCH)
    assert not oracle_equals_gemm(plan, cmds, modes=("max",))


def test_wrong_weight_retention_across_k_rejected():
    """tests/test_gemmini_general.py:37-45."""
    plan = sc.make_plan(32, 16, 32, "reuse_b")
    cmds = copy.deepcopy(sc.gen_commands(plan))
    for index, c in enumerate(cmds):
        if c["kind"] == "preload" and c["out_addr"] & sc.ACCUMULATE_BIT:
            c["bd_spad_addr"] = sc.GARBAGE_ADDR
            cmds[index + 1]["accumulated"] = True
            break
    assert not sc.check_program(plan, cmds)[0]


def test_batched_reuse_handles_partial_last_batch():
    """tests/test_gemmini_general.py:47-57."""
    plan = sc.make_plan(48, 16, 32, "baseline")
    plan["accumulator_rows"] = 32
    cmds = sc.gen_batched_reuse_b(plan, 2)
    assert sc.check_program(plan, cmds)[:2] == (True, "accepted")
    assert sc.modeled_counts(cmds)["mvin_B"] == 4
    assert oracle_equals_gemm(plan, cmds)


def test_overlarge_batch_is_rejected_by_execution():
    """tests/test_gemmini_general.py:59-66: a batch of 3 needs 48 accumulator
    rows of a plan that has 32."""
    plan = sc.make_plan(48, 16, 32, "baseline")
    plan["accumulator_rows"] = 32
    ok, why, _ = sc.check_program(plan, sc.gen_batched_reuse_b(plan, 3))
    assert not ok and "execution rejected" in why


def test_zero_batch_and_invalid_plans_raise():
    """tests/test_gemmini_general.py:68-70."""
    with pytest.raises(ValueError):
        sc.gen_batched_reuse_b(sc.make_plan(16, 16, 16, "baseline"), 0)
    with pytest.raises(ValueError):
        sc.gen_batched_reuse_b(sc.make_plan(16, 16, 16, "baseline"), True)
    with pytest.raises(ValueError):
        sc.gen_batched_reuse_b(sc.make_plan(16, 16, 24, "baseline"), 1)


def test_missing_fence_and_product_order_are_refused():
    plan = sc.make_plan(16, 16, 32, "baseline")
    cmds = sc.gen_commands(plan)
    assert sc.check_program(plan, cmds[:-1]) == (False, sc.NOT_DRAINED, None)
    # The two k steps swapped: the same sum mod 2^32, but not the product
    # sequence the specification fixes (Symbolic.lean:30-34 compares lists).
    body = cmds[4:-2]
    swapped = copy.deepcopy(cmds[:4] + body[4:] + body[:4] + cmds[-2:])
    swapped[6]["out_addr"] &= ~sc.ACCUMULATE_BIT
    swapped[10]["out_addr"] |= sc.ACCUMULATE_BIT
    assert oracle_equals_gemm(plan, swapped, modes=("lcg",))
    ok, why, _ = sc.check_program(plan, swapped)
    assert not ok and why.startswith(sc.OUTPUT_MISMATCH)


def _mutants(cmds, rng, count):
    fields = ("offset", "spad_addr", "out_addr", "acc_addr", "buf_offset", "a_spad_addr",
              "bd_spad_addr", "accumulated", "stride_bytes")
    for _ in range(count):
        c = copy.deepcopy(cmds)
        i = rng.randrange(len(c))
        how = rng.randrange(4)
        if how == 0:
            del c[i]
        elif how == 1 and i + 1 < len(c):
            c[i], c[i + 1] = c[i + 1], c[i]
        else:
            keys = [f for f in fields if f in c[i]]
            if not keys:
                continue
            f = rng.choice(keys)
            v = c[i][f]
            if isinstance(v, bool):
                c[i][f] = not v
            elif f in ("out_addr", "acc_addr") and rng.random() < 0.5:
                c[i][f] = v ^ sc.ACCUMULATE_BIT
            else:
                c[i][f] = v + rng.choice((-16, 16, 1))
        yield c


def test_every_stream_the_check_accepts_computes_the_gemm():
    """Soundness against the oracle interpreter: single-command mutations
    (deleted, swapped with the next, one field moved) of generated streams
    are either refused or compute exactly the GEMM on two inputs."""
    rng = random.Random(5)
    refused = accepted = 0
    for m, n, k in ((32, 32, 32), (48, 16, 32)):
        for plan, cmds in ((sc.make_plan(m, n, k, "baseline"), None),
                           (sc.make_plan(m, n, k, "reuse_b"), None)):
            cmds = sc.gen_commands(plan)
            for mut in _mutants(cmds, rng, 150):
                ok = sc.check_program(plan, mut)[0]
                if not ok:
                    refused += 1
                    continue
                accepted += 1
                assert oracle_equals_gemm(plan, mut, seed=3, modes=("lcg", "minmax"))
    assert refused > 300 and accepted > 0


def test_malformed_commands_are_refused_not_raised():
    plan = sc.make_plan(16, 16, 16, "baseline")
    cmds = sc.gen_commands(plan)
    for bad in (dict(cmds[7], a_spad_addr=[0]), dict(cmds[6], out_addr=None),
                {k: v for k, v in cmds[4].items() if k != "spad_addr"}, "mvin", None):
        mutated = cmds[:4] + [bad] + cmds[5:]
        ok, why, _ = sc.check_program(plan, mutated)
        assert not ok and why.startswith(sc.EXECUTION_REJECTED), (bad, why)
    assert not sc.check_program(plan, "not a list")[0]
    assert not sc.check_program({"m": 16}, cmds)[0]


def test_accepted_receipt_and_reference_return_shape():
    plan = sc.make_plan(32, 32, 32, "reuse_b")
    ok, why, receipt = sc.check_program(plan, sc.gen_commands(plan))
    assert ok and why == "accepted"
    assert receipt["cells"] == 32 * 32 and receipt["products_per_cell"] == 32


def _mutated(schedule, m, n, k, mutate):
    plan = sc.make_plan(m, n, k, schedule)
    cmds = copy.deepcopy(sc.gen_commands(plan))
    mutate(cmds)
    return plan, cmds


def _first(cmds, kind, **fields):
    return next(c for c in cmds if c["kind"] == kind and all(c[f] == v for f, v in fields.items()))


def _bump(cmd, field, by):
    cmd[field] += by


def _drop_last(cmds, kind):
    del cmds[max(i for i, x in enumerate(cmds) if x["kind"] == kind)]


# The command-level mutations of the reference's tests/test_gemmini_program.py
# (:95-171, :261-281): each must be refused by the check alone. The
# reference's byte-encoding mutations, and the trailing duplicate fence and
# the swap of the two leading configuration commands (:161-171), are refused
# there by the binding of commands to executable bytes; the command streams
# they leave still compute the GEMM, so the check accepts them.
PROGRAM_MUTATIONS = {
    "mvin A offset + 16": lambda c: _bump(_first(c, "mvin", slot=0), "offset", 16),
    "mvin B offset + 8": lambda c: _bump(_first(c, "mvin", slot=1), "offset", 8),
    "A stride + 1": lambda c: _bump(_first(c, "config_ld", slot=0), "stride_bytes", 1),
    "accumulate flag flipped": lambda c: _bump(_first(c, "preload"), "out_addr", sc.ACCUMULATE_BIT),
    "preload source dropped": lambda c: _first(c, "preload").update(bd_spad_addr=sc.GARBAGE_ADDR),
    "missing fence": lambda c: _drop_last(c, "fence"),
    "missing mvout": lambda c: _drop_last(c, "mvout"),
    "unknown op": lambda c: c.insert(0, {"kind": "flush"}),
    "out of bound memory": lambda c: _first(c, "mvin", buf="A").update(offset=10 ** 9),
    "output-stationary dataflow": lambda c: _first(c, "config_ex").update(dataflow=0),
}


@pytest.mark.parametrize("name", sorted(PROGRAM_MUTATIONS))
@pytest.mark.parametrize("shape", [(16, 16, 16), (64, 64, 64)])
def test_reference_program_mutations_are_refused(name, shape):
    plan, cmds = _mutated("baseline", *shape, PROGRAM_MUTATIONS[name])
    assert not sc.check_program(plan, cmds)[0], (name, shape)


def test_retained_compute_turned_preloaded_is_refused():
    """tests/test_gemmini_program.py:125-130: a reuse_b compute that retains
    B, turned into one that latches it, has no B source to latch."""
    plan = sc.make_plan(32, 16, 16, "reuse_b")
    cmds = copy.deepcopy(sc.gen_commands(plan))
    assert sc.check_program(plan, cmds)[0]
    _first(cmds, "compute", accumulated=True)["accumulated"] = False
    assert not sc.check_program(plan, cmds)[0]


def test_byte_bound_mutations_leave_the_gemm():
    """The two command mutations the reference refuses only through the
    executable bytes compute the GEMM, and the check accepts them."""
    plan = sc.make_plan(16, 16, 16, "baseline")
    cmds = sc.gen_commands(plan)
    for mutated in (cmds + [copy.deepcopy(cmds[-1])], [cmds[1], cmds[0]] + cmds[2:]):
        assert sc.check_program(plan, mutated)[:2] == (True, "accepted")
        assert oracle_equals_gemm(plan, mutated, modes=("lcg", "minmax"))
